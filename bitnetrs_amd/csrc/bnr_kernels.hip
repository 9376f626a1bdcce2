// bnr_kernels.hip -- gfx950 kernels of the GQA attention hot path.
//
//  rope_append_kernel  half-split RoPE of q/k + head-major KV append
//                       (rope_append_vec_kernel: four pairs per thread)
//  decode_kernel<G,RPG> split-K decode attention, head_dim 128, optional
//                       fused RoPE + append, last-workgroup merge
//  decode_generic_kernel any head_dim / group size
//
// Wave64 throughout.  The decode kernel reads each K/V row of a kv head once
// and serves the G query heads of the group from registers (the reference
// re-reads every row once per query head, bitnet-cpu/src/attention.rs:
// 170-204).
#include <type_traits>

#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

namespace bnr {
namespace {

// ---------------------------------------------------------------------------
// RoPE rotation of one half-split pair, exactly as apply_rope_to_head_slice
// (bitnet-cpu/src/rope.rs:414-430): two rounded products, then one rounded
// add/sub.  Contraction is off so the result is bit-identical to the
// reference's f32 arithmetic.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void rot_pair(float lo, float hi, float c, float s, float &olo,
                                         float &ohi) {
#pragma clang fp contract(off)
  olo = lo * c - hi * s;
  ohi = hi * c + lo * s;
}

__device__ __forceinline__ void rot4(float4 lo, float4 hi, float4 c, float4 s, float4 &olo,
                                     float4 &ohi) {
  rot_pair(lo.x, hi.x, c.x, s.x, olo.x, ohi.x);
  rot_pair(lo.y, hi.y, c.y, s.y, olo.y, ohi.y);
  rot_pair(lo.z, hi.z, c.z, s.z, olo.z, ohi.z);
  rot_pair(lo.w, hi.w, c.w, s.w, olo.w, ohi.w);
}

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
}

// ---------------------------------------------------------------------------
// Cross-lane helpers (DPP inside a 16-lane row).
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row gets the total.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Max / sum over the 16 lanes of a DPP row (every lane of the row gets it).
__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  v = fmaxf(v, dpp<0x140>(v));
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Wave-uniform max / sum over 64 lanes: DPP inside each row, then the four
// row results through readlane.
__device__ __forceinline__ float wave_max(float v) {
  v = row_max16(v);
  return fmaxf(fmaxf(readlane(v, 0), readlane(v, 16)), fmaxf(readlane(v, 32), readlane(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  return (readlane(v, 0) + readlane(v, 16)) + (readlane(v, 32) + readlane(v, 48));
}

__device__ __forceinline__ float dot8(float4 alo, float4 ahi, float4 blo, float4 bhi) {
  float d = alo.x * blo.x;
  d = fmaf(alo.y, blo.y, d);
  d = fmaf(alo.z, blo.z, d);
  d = fmaf(alo.w, blo.w, d);
  d = fmaf(ahi.x, bhi.x, d);
  d = fmaf(ahi.y, bhi.y, d);
  d = fmaf(ahi.z, bhi.z, d);
  d = fmaf(ahi.w, bhi.w, d);
  return d;
}

__device__ __forceinline__ float4 axpy4(float a, float4 x, float4 y) {
  return make_float4(fmaf(a, x.x, y.x), fmaf(a, x.y, y.y), fmaf(a, x.z, y.z),
                     fmaf(a, x.w, y.w));
}

__device__ __forceinline__ float4 scale4(float a, float4 x) {
  return make_float4(a * x.x, a * x.y, a * x.z, a * x.w);
}

__device__ __forceinline__ float4 ld4(const float *p) {
  return *reinterpret_cast<const float4 *>(p);
}

__device__ __forceinline__ void st4(float *p, float4 v) {
  *reinterpret_cast<float4 *>(p) = v;
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
}

// Agent-coherent scalar store / load: performed at the device-wide coherence
// point, so another workgroup -- on any XCD, behind its own L2 -- that reads
// after observing the ticket below sees the value without a cache writeback
// or invalidate of the whole L2.
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
      klo[i] = ld4(kc + off + 4 * j);
      khi[i] = ld4(kc + off + 64 + 4 * j);
    }
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const long long off = (long long)(valid[i] ? tp + i * 16 + rg : t0) * D;
      vlo[i] = ld4(vc + off + 4 * j);
      vhi[i] = ld4(vc + off + 64 + 4 * j);
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
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
        if (tp + i * 16 + rg == pos) {
          klo[i] = nklo;
          khi[i] = nkhi;
          vlo[i] = nvlo;
          vhi[i] = nvhi;
          st4(kc + (long long)pos * D + 4 * j, nklo);
          st4(kc + (long long)pos * D + 64 + 4 * j, nkhi);
          st4(vc + (long long)pos * D + 4 * j, nvlo);
          st4(vc + (long long)pos * D + 64 + 4 * j, nvhi);
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
// Causal flash prefill on the fp32 matrix cores (v_mfma_f32_32x32x2_f32).
//
// Workgroup = one kv head's G query heads (one wave each) x 32 queries; the
// G waves share every 32-key K/V tile.  Tiles go from HBM straight into LDS
// (global_load_lds, 16 bytes per lane, no staging registers), double
// buffered in four separate LDS arrays so that the compiler can tell a read
// of the current tile from the copy of the next one still in flight.  The
// register budget (at most 256 per lane) lets two workgroups share a CU:
// one's softmax, LDS reads and start-up run under the other's MFMAs.
//
// Each wave computes S^T = K Q^T (32 keys x 32 queries), so the accumulator
// layout of S^T is exactly the B-operand layout P^T needs for O^T = V^T P^T:
// no transposes, no LDS round trip for P.
//
// Lane l of a wave: col = l % 32 is its query, hl = l / 32 its half.  Q
// fragment: dims 64*hl .. 64*hl+63 of that query (registers, prescaled by
// log2(e)/sqrt(d)).  MFMA step kk (0..63) uses dim 64*hl + kk for the lane's
// k-slot, so K rows are read from LDS as float4s; K rows are stored with
// their 16-byte chunks XOR-swizzled by (row % 16) so that the 32 rows read
// at one step fall in distinct banks.  Accumulator register r of a 32x32
// tile holds row 8*(r/4) + 4*hl + r%4.  In O^T, row i of dim block db is
// head dim 4*i + db, so the four values a lane needs for one PV step are
// the float4 at dims 4*col of one V row, unpermuted.  Online softmax per
// query: a key tile's max and sum are the lane's 16 values plus its partner
// lane l^32.
//
// Long query tiles are cut into key chunks of chunk_tiles tiles (separate
// workgroups); the last chunk of a tile to finish merges the others' partial
// states.  Work items are dispatched longest query tile first.
// ---------------------------------------------------------------------------
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// 16 bytes per lane from global memory straight into LDS: lane i of the wave
// writes bytes [16 i, 16 i + 16) after `lds`, which must be wave-uniform.
__device__ __forceinline__ void dma16(const float *g, float *lds) {
  __builtin_amdgcn_global_load_lds((global_void_t *)g, (lds_void_t *)lds, 16, 0, 0);
}

// s_waitcnt vmcnt(0) alone (expcnt and lgkmcnt at their maxima).
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Two waves per SIMD: at most 256 registers per lane.  (G = 2 reaches only
// one: two of its workgroups fill LDS.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Wpass-failed"
constexpr int kPrefillTile = 32 * kHeadDim;  // floats per K (or V) tile

// A prefill work item: kv head h, item y -> (query tile qt, key chunk ch of
// nch), key tiles kt0 .. nkt-1, partial-state slot of the tile's chunk 0
// (base).  The order of the items is prefill_map's.
struct PfItem {
  int h, y, qt, ch, nch, base, q0, kt0, nkt;
};

__device__ __forceinline__ PfItem pf_item(const PrefillArgs &a, int h, int y) {
  PfItem it;
  it.h = h;
  it.y = y;
  const int last_row = a.start_pos + a.n_tokens - 1;
  prefill_map(a, y, it.qt, it.ch, it.nch, it.base);
  it.q0 = it.qt * 32;
  const int kmax = min(a.start_pos + it.q0 + 31, last_row);
  it.kt0 = it.ch * a.chunk_tiles;
  it.nkt = min(kmax / 32 + 1, it.kt0 + a.chunk_tiles);
  return it;
}

// Copy of key tile kt of kv head h: copy j of wave w fills rows 2J, 2J+1
// (J = w*NI + j); lane l takes row 2J + l/32, LDS chunk l%32.  Rows past the
// last cached one repeat it (their keys are masked for every query).
template <int G>
__device__ __forceinline__ void pf_copy_tile(const PrefillArgs &a, int h, int kt, float *dk,
                                             float *dv) {
  constexpr int NI = kPrefillTile / 4 / (64 * G);  // 1 KB copies per wave per tile
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int last_row = a.start_pos + a.n_tokens - 1;
  const float *kc = a.k_cache + h * a.kv_stride;
  const float *vc = a.v_cache + h * a.kv_stride;
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int J = wave * NI + j;
    const int r = 2 * J + hl, p = col;
    const long long grow = (long long)min(kt * 32 + r, last_row) * kHeadDim;
    dma16(kc + grow + 4 * (p ^ (r & 15)), dk + J * 256);
    dma16(vc + grow + 4 * p, dv + J * 256);
  }
}

// This lane's Q fragment (dims 64*hl .. 64*hl+63 of its query, the wave's
// head), unscaled.
template <int G>
__device__ __forceinline__ void pf_load_q(const PrefillArgs &a, const PfItem &it, float (&qf)[64]) {
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qrow = min(it.q0 + col, a.n_tokens - 1);  // rows past the end are not stored
  const float *qp = a.q + ((long long)qrow * a.n_heads + it.h * G + g) * kHeadDim + 64 * hl;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 v = ld4(qp + 4 * i);
    qf[4 * i] = v.x;
    qf[4 * i + 1] = v.y;
    qf[4 * i + 2] = v.z;
    qf[4 * i + 3] = v.w;
  }
}

__device__ __forceinline__ void pf_scale_q(float (&qf)[64], float sc) {
#pragma unroll
  for (int i = 0; i < 64; ++i) qf[i] *= sc;
}

// S^T tile = K Q^T: 32 keys x 32 queries.
__device__ __forceinline__ floatx16 pf_tile_s(const float *dk, const float (&qf)[64]) {
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  floatx16 S = floatx16{};
  const float *krow = dk + col * kHeadDim + 64 * hl;
  const int sw = col & 15;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 kv = ld4(krow + 4 * (i ^ sw));
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * i], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * i + 1], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * i + 2], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * i + 3], S, 0, 0, 0);
  }
  return S;
}

// Causal mask, online softmax and O^T += V^T P^T for key tile kt.
__device__ __forceinline__ void pf_tile_pv(const PrefillArgs &a, const PfItem &it, int kt,
                                           floatx16 S, const float *dv, floatx16 (&O)[4],
                                           float &m, float &l) {
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  const int kbase = kt * 32;
  if (kbase + 31 > a.start_pos + it.q0) {  // the tile reaches the causal diagonal
    const int pq = a.start_pos + min(it.q0 + col, a.n_tokens - 1);  // this lane's query position
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kbase + 8 * (r >> 2) + 4 * hl + (r & 3);
      if (key > pq) S[r] = -INFINITY;
    }
  }
  float mb = S[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) mb = fmaxf(mb, S[r]);
  mb = fmaxf(mb, __shfl_xor(mb, 32));
  // Lazy rescaling: m is the reference the exponentials are taken against;
  // it moves only when a query's max exceeds it by more than 8 (so every
  // p <= 2^8).  O lives in accumulation registers, so a rescale is costly
  // and is skipped for the whole wave when no lane needs it.  The first
  // tile with a visible key sets m.
  if (__ballot(mb > m + 8.0f) != 0) {
    const float mn = fmaxf(m, mb);
    const float alpha = fast_exp2(m - mn);
    l *= alpha;
#pragma unroll
    for (int db = 0; db < 4; ++db) O[db] *= alpha;
    m = mn;
  }
  float p[16], ls = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    p[r] = fast_exp2(S[r] - m);
    ls += p[r];
  }
  l += ls;
  // O^T += V^T P^T: step s takes key row 8*(s/4) + 4*hl + s%4 of the tile.
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float4 vv = ld4(dv + (8 * (s >> 2) + 4 * hl + (s & 3)) * kHeadDim + 4 * col);
    O[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.x, p[s], O[0], 0, 0, 0);
    O[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.y, p[s], O[1], 0, 0, 0);
    O[2] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.z, p[s], O[2], 0, 0, 0);
    O[3] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv.w, p[s], O[3], 0, 0, 0);
  }
}

// End of an item: a chunk of a split query tile stores its partial state and
// takes a ticket; the last chunk to finish merges the others into its own
// registers and, like an unsplit item, writes the output.
template <int G>
__device__ __forceinline__ void pf_finish(const PrefillArgs &a, const PfItem &it,
                                          floatx16 (&O)[4], float m, float l, int *s_last) {
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, col = lane & 31;
  const int g = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = it.h, head = h * G + g;
  if (it.nch > 1) {
    // Partial state of this chunk, lane-coalesced: component c (0..63 O, 64 m,
    // 65 l) of lane `lane` of wave g at ws[((item * G + g) * 66 + c) * 64 + lane].
    float *slot = a.ws + (((long long)h * a.n_items + it.base + it.ch) * G + g) * 66 * 64 + lane;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st_agent(slot + (16 * db + r) * 64, O[db][r]);
    st_agent(slot + 64 * 64, m);
    st_agent(slot + 65 * 64, l);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
    __syncthreads();
    unsigned *ctr = a.counters + ((long long)h * a.n_qtiles + it.qt) * kCounterStride;
    if (tid == 0) {
      const unsigned ticket =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = ticket == (unsigned)(it.nch - 1);
    }
    __syncthreads();
    const bool last = *s_last;
    __syncthreads();  // s_last is read before the next item may write it
    if (!last) return;
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Merge the other chunks into this one's registers (same lane layout).
    for (int c = 0; c < it.nch; ++c) {
      if (c == it.ch) continue;
      const float *src = a.ws + (((long long)h * a.n_items + it.base + c) * G + g) * 66 * 64 + lane;
      float ov[64];
#pragma unroll
      for (int i = 0; i < 64; ++i) ov[i] = ld_agent(src + i * 64);
      const float mc = ld_agent(src + 64 * 64), lc = ld_agent(src + 65 * 64);
      const float mn = fmaxf(m, mc);
      const float sa = fast_exp2(m - mn), sb = fast_exp2(mc - mn);
      l = l * sa + lc * sb;
      m = mn;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int r = 0; r < 16; ++r) O[db][r] = O[db][r] * sa + ov[16 * db + r] * sb;
    }
  }
  // Lane (col, hl) holds, for r = 4*rq + r3, dims 32*rq + 16*hl + 4*r3 + db.
  const float inv = 1.0f / (l + __shfl_xor(l, 32));
  if (it.q0 + col < a.n_tokens) {
    float *op = a.out + ((long long)(it.q0 + col) * a.n_heads + head) * kHeadDim + 16 * hl;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      st4(op + 32 * (r >> 2) + 4 * (r & 3),
          make_float4(O[0][r] * inv, O[1][r] * inv, O[2][r] * inv, O[3][r] * inv));
  }
}

// Grid-mapped prefill: workgroup (h = blockIdx.x, y = blockIdx.y), kv head
// the fastest axis, so the longest items of every head are dispatched first.
// The four LDS tile buffers are separate arrays so that the compiler can
// tell a read of the current tile from the copy of the next one in flight.
template <int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float sK0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sK1[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV1[kPrefillTile];
  __shared__ int s_last;
  const PfItem it = pf_item(a, blockIdx.x, blockIdx.y);
  pf_copy_tile<G>(a, it.h, it.kt0, sK0, sV0);
  float qf[64];
  pf_load_q<G>(a, it, qf);
  pf_scale_q(qf, a.scale_log2);
  wait_vmem();
  __syncthreads();
  floatx16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = floatx16{};
  // m starts finite: in a chunk that is not the first, a query may see no key
  // at all (p = 0 for it throughout, and no -inf - -inf in the rescale).
  float m = -1e30f, l = 0.f;
  auto step = [&](int kt, const float *dk, const float *dv, float *nk, float *nv) {
    if (kt + 1 < it.nkt) pf_copy_tile<G>(a, it.h, kt + 1, nk, nv);
    const floatx16 S = pf_tile_s(dk, qf);
    pf_tile_pv(a, it, kt, S, dv, O, m, l);
    wait_vmem();  // this wave's copies of the next tile have landed
    __syncthreads();
  };
  for (int kt = it.kt0;;) {
    step(kt, sK0, sV0, sK1, sV1);
    if (++kt >= it.nkt) break;
    step(kt, sK1, sV1, sK0, sV0);
    if (++kt >= it.nkt) break;
  }
  pf_finish<G>(a, it, O, m, l, &s_last);
}

// Persistent prefill: gridDim.x resident workgroups (at most the number of
// items) start on item blockIdx.x and take further items (kv head fastest,
// longest first) from an atomic queue.  The next item's index is taken
// during the current item's first tile; during its last tile the next
// item's first K/V tile is copied into the free buffer pair and, once the
// tile's products have read the Q fragment, the next Q fragment is loaded,
// so a workgroup's start-up latency runs under the previous item's work.
// (After a one-tile item the successor is loaded without overlap: its index
// arrives with that tile.)  Tiles alternate between the two buffer pairs
// across item boundaries; the loop body is unrolled over the pair so that
// each buffer is named statically (the compiler can tell the copy in flight
// from the tile being read).  A workgroup leaves once its queue index passes
// the last item; the last to leave resets the queue for the next launch.
template <int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_persistent_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float sK0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sK1[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV1[kPrefillTile];
  __shared__ int s_last, s_item[2];
  const int tid = threadIdx.x;
  const int total = a.n_kv * a.n_items;
  unsigned *next = a.queue, *left = a.queue + kCounterStride;
  auto item = [&](int y) { return pf_item(a, y % a.n_kv, y / a.n_kv); };
  PfItem it = item(blockIdx.x);
  pf_copy_tile<G>(a, it.h, it.kt0, sK0, sV0);
  float qf[64];
  pf_load_q<G>(a, it, qf);
  pf_scale_q(qf, a.scale_log2);
  wait_vmem();
  __syncthreads();
  floatx16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = floatx16{};
  float m = -1e30f, l = 0.f;
  int kt = it.kt0, par = 0;
  int nxt = total;  // the next item, once its index has arrived
  // One tile on (dk, dv); the next tile of this item, or the next item's
  // first, is copied into (nk, nv).  Returns false once the workgroup has no
  // item left.
  auto step = [&](const float *dk, const float *dv, float *nk, float *nv) -> bool {
    const bool first = kt == it.kt0, lastt = kt + 1 == it.nkt;
    const bool pre = lastt && nxt < total;
    PfItem nit = pre ? item(nxt) : it;
    if (!lastt || pre) pf_copy_tile<G>(a, lastt ? nit.h : it.h, lastt ? nit.kt0 : kt + 1, nk, nv);
    int ticket = 0;
    if (first && tid == 0)  // in flight during this tile
      ticket = (int)gridDim.x +
               (int)__hip_atomic_fetch_add(next, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const floatx16 S = pf_tile_s(dk, qf);
    pf_tile_pv(a, it, kt, S, dv, O, m, l);
    if (pre) pf_load_q<G>(a, nit, qf);  // qf is no longer read by this item
    if (first && tid == 0) s_item[par] = ticket;
    if (lastt) pf_finish<G>(a, it, O, m, l, &s_last);
    wait_vmem();  // this wave's copies (next tile, next Q) have landed
    __syncthreads();
    // The slot alternates with the item: a rewrite of one slot comes after
    // the following item's first barrier, which every reader has passed.
    if (first) nxt = __builtin_amdgcn_readfirstlane(s_item[par]);
    if (!lastt) {
      ++kt;
      return true;
    }
    if (nxt >= total) return false;
    if (!pre) {  // one-tile item: the successor was not known in time
      nit = item(nxt);
      pf_copy_tile<G>(a, nit.h, nit.kt0, nk, nv);
      pf_load_q<G>(a, nit, qf);
      wait_vmem();
      __syncthreads();
    }
    it = nit;
    kt = it.kt0;
    nxt = total;
    par ^= 1;
    pf_scale_q(qf, a.scale_log2);
#pragma unroll
    for (int db = 0; db < 4; ++db) O[db] = floatx16{};
    m = -1e30f;
    l = 0.f;
    return true;
  };
  for (;;) {
    if (!step(sK0, sV0, sK1, sV1)) break;
    if (!step(sK1, sV1, sK0, sV0)) break;
  }
  if (tid == 0) {
    const unsigned out = __hip_atomic_fetch_add(left, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (out == gridDim.x - 1) {  // every workgroup has taken its last index
      __hip_atomic_store(next, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(left, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}
#pragma clang diagnostic pop

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
  return a.merge_inline ? launch_decode_gi<G, true>(a, s) : launch_decode_gi<G, false>(a, s);
}

}  // namespace

hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t s) {
  auto a16 = [](const void *p) { return ((uintptr_t)p & 15) == 0; };
  const int half = a.head_dim / 2;
  const bool vec = half % 4 == 0 && a16(a.q) && a16(a.k) && a16(a.cos_tab) && a16(a.sin_tab) &&
                   (!a.v_cache || (a16(a.v) && a16(a.v_cache))) && (!a.k_cache || a16(a.k_cache)) &&
                   a.kv_stride % 4 == 0;
  const long long total = (long long)a.n_tokens * (a.n_heads + 2 * a.n_kv) * (vec ? half / 4 : half);
  if (total == 0) return hipSuccess;
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
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

bool prefill_supported(int group) { return group == 2 || group == 4 || group == 8; }

void prefill_order(PrefillArgs &a) {
  const int ct = a.chunk_tiles, nqt = a.n_qtiles;
  const int last_row = a.start_pos + a.n_tokens - 1;
  const int A = (a.start_pos + 31) / 32 + 1;
  const int nt_last = last_row / 32 + 1;
  a.lpt = ct <= kMaxLptChunk && ct > 1;
  a.n_full = 0;
  for (int b = 0; b < kMaxLptChunk; ++b) a.part_off[b] = 0;
  if (!a.lpt) return;
  int count[kMaxLptChunk] = {};  // last chunks of length r (< ct)
  a.n_full = nt_last / ct;
  count[nt_last % ct] += 1;
  for (int qt = 0; qt + 1 < nqt; ++qt) {
    a.n_full += (qt + A) / ct;
    count[(qt + A) % ct] += 1;
  }
  // bucket b holds length ct-1-b; part_off[b] = items of longer buckets
  for (int b = 1; b < ct; ++b) a.part_off[b] = a.part_off[b - 1] + count[ct - b];
}

PrefillPlan prefill_plan(int n_tokens, int start_pos, int chunk_tiles) {
  const int last_row = start_pos + n_tokens - 1, nqt = (n_tokens + 31) / 32;
  const int ctiles = chunk_tiles;
  PrefillPlan p{0, 0, false};
  for (int qt = 0; qt < nqt; ++qt) {
    const int nk = std::min(start_pos + qt * 32 + 31, last_row) / 32 + 1;
    const int nch = (nk + ctiles - 1) / ctiles;
    p.n_items += nch;
    p.key_tiles += nk;
    p.split |= nch > 1;
  }
  return p;
}

hipError_t launch_prefill(const PrefillArgs &a, int group, int persistent_wgs, hipStream_t s) {
  if (a.n_tokens <= 0) return hipSuccess;
  if (persistent_wgs > 0) {
    if (!a.queue) return hipErrorInvalidValue;
    const dim3 grid(persistent_wgs);
    switch (group) {
      case 2: prefill_persistent_kernel<2><<<grid, dim3(128), 0, s>>>(a); break;
      case 4: prefill_persistent_kernel<4><<<grid, dim3(256), 0, s>>>(a); break;
      case 8: prefill_persistent_kernel<8><<<grid, dim3(512), 0, s>>>(a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const dim3 grid(a.n_kv, a.n_items);
  switch (group) {
    case 2: prefill_kernel<2><<<grid, dim3(128), 0, s>>>(a); break;
    case 4: prefill_kernel<4><<<grid, dim3(256), 0, s>>>(a); break;
    case 8: prefill_kernel<8><<<grid, dim3(512), 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode_generic(const DecodeGenericArgs &a, hipStream_t s) {
  decode_generic_kernel<<<dim3(a.n_heads), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace bnr
