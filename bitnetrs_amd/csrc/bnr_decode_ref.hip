// bnr_decode_ref.hip -- gfx950 split-K decode attention with the reference
// merge (decode_reg_kernel): splits weigh their rows against the score of the
// newest row and accumulate with device-scope atomics.
#include "bnr_device.h"
#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

namespace bnr {
namespace {

// Device-scope atomic reads.  A read-modify-write always reads the last
// value of its location's modification order, wherever the lines of that
// location are cached, so the merge needs no cache maintenance.
__device__ __forceinline__ float take_f32(float *p) {  // read and clear
  return __hip_atomic_exchange(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 take_f32x2(float *p) {  // two adjacent floats, read and clear
  return __builtin_bit_cast(
      float2, __hip_atomic_exchange(reinterpret_cast<unsigned long long *>(p), 0ull,
                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}
__device__ __forceinline__ unsigned long long take_u64(float *p) {
  return __hip_atomic_exchange(reinterpret_cast<unsigned long long *>(p), 0ull, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float read_rmw(const float *p) {  // read, leave in place
  return __hip_atomic_fetch_add(const_cast<float *>(p), 0.f, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
}

// The last workgroup of (sequence b, kv head h): one batch of atomic
// exchanges that read the output sums, the weight sums and the masks and
// leave zeros for the next launch; then the division.  Splits flagged in
// the masks kept their own maximum and are folded in first.  R: the
// reference scores; s_L (G floats) and s_mk (4 words): LDS.
template <int G>
__device__ __forceinline__ void ref_merge(const DecodeArgs &a, int b, int h, float *acc,
                                          const float *R, float *s_L, unsigned long long *s_mk,
                                          int tid, int nthreads) {
  constexpr int D = kHeadDim;
  constexpr int NE2 = G * D / 2;  // pairs of outputs
  float2 o2[(NE2 + 255) / 256];
#pragma unroll
  for (int k = 0; k < (NE2 + 255) / 256; ++k) {
    const int e2 = tid + k * nthreads;
    if (e2 < NE2) o2[k] = take_f32x2(acc + 2 * e2);
  }
  if (tid < G) s_L[tid] = take_f32(acc + kAccL + tid);
  if (tid >= 64 && tid < 68) s_mk[tid - 64] = take_u64(acc + kAccMask + 2 * (tid - 64));
  __syncthreads();
  const bool flagged = (s_mk[0] | s_mk[1] | s_mk[2] | s_mk[3]) != 0;
#pragma unroll
  for (int k = 0; k < (NE2 + 255) / 256; ++k) {
    const int e2 = tid + k * nthreads;
    if (e2 >= NE2) continue;
    const int e = 2 * e2, g = e / D;
    float O[2] = {o2[k].x, o2[k].y};
    float Ls = s_L[g];
    if (flagged) {
      float M = Ls > 0.f ? R[g] : -INFINITY;
      for (int i = 0; i < 4; ++i) {
        for (unsigned long long bits = s_mk[i]; bits; bits &= bits - 1) {
          const long long sp = a.split_off[b] + 64 * i + __builtin_ctzll(bits);
          const float *ml = reinterpret_cast<const float *>(&a.ws_ml[(sp * a.n_kv + h) * G + g]);
          const float ms = read_rmw(ml), ls = read_rmw(ml + 1);
          if (!(ms > -INFINITY)) continue;  // no valid row in that split
          const float *po = &a.ws_o[(sp * a.n_kv + h) * G * D + e];
          const float os0 = read_rmw(po), os1 = read_rmw(po + 1);
          const float mn = fmaxf(M, ms);
          const float wa = M == -INFINITY ? 0.f : fast_exp2(M - mn), wb = fast_exp2(ms - mn);
          Ls = Ls * wa + ls * wb;
          O[0] = O[0] * wa + os0 * wb;
          O[1] = O[1] * wa + os1 * wb;
          M = mn;
        }
      }
    }
    float *op = a.out + b * a.out_bstride + (long long)h * G * D + e;
    *reinterpret_cast<float2 *>(op) = make_float2(O[0] / Ls, O[1] / Ls);
  }
}

// The deterministic form of the merge (merge_det): every split stored its
// (m, l, O) -- m = R for a split on the reference path, its own maximum on
// the exact path -- with agent-scope stores, and the last workgroup of
// (sequence b, kv head h) combines them in a fixed order: the maxima and
// weights w_s = exp2(m_s - M) in a fixed tree, then for every output the
// splits in split order.  When every split used the reference, every w_s is
// exp2(0) = 1 and the result is a sum in a fixed order.  The bits of the
// output do not depend on the order in which the splits finished.  s_ml:
// LDS for nsplit * G (m, l) pairs; s_wt: LDS for kMaxSplits * G weights,
// then one float4 per thread.
template <int G>
__device__ __forceinline__ void det_merge(const DecodeArgs &a, int b, int h, int nsplit,
                                          float2 *s_ml, float *s_wt, float *s_L, int tid,
                                          int nthreads) {
  constexpr int D = kHeadDim;
  const long long s0 = a.split_off[b];
  for (int i = tid; i < nsplit * G; i += nthreads) {  // i = s * G + g
    const float *ml = reinterpret_cast<const float *>(&a.ws_ml[((s0 + i / G) * a.n_kv + h) * G + i % G]);
    s_ml[i] = make_float2(ld_agent(ml), ld_agent(ml + 1));
  }
  __syncthreads();
  // wave g: the maximum over the splits, then the weights and the weight sum
  // (lane-strided partial sums, then a fixed tree over the lanes)
  const int wave = tid >> 6, lane = tid & 63;
  if (wave < G) {
    const int g = wave;
    float M = -INFINITY;
    for (int sp = lane; sp < nsplit; sp += 64) M = fmaxf(M, s_ml[sp * G + g].x);
    M = wave_max(M);
    float Lp = 0.f;
    for (int sp = lane; sp < nsplit; sp += 64) {
      const float2 v = s_ml[sp * G + g];
      const float wgt = v.x > -INFINITY ? fast_exp2(v.x - M) : 0.f;
      s_wt[sp * G + g] = wgt;
      Lp = fmaf(wgt, v.y, Lp);
    }
    const float Ls = wave_sum(Lp);
    if (lane == 0) s_L[g] = Ls;
  }
  __syncthreads();
  // Thread t: the float4 of outputs 4 q4 .. 4 q4 + 3 (q4 = t % NQ), over
  // the splits sp = sg, sg + NSG, ... in order (sg = t / NQ), with 16-byte
  // agent-scope loads (buffer loads with sc1); then the NSG partial sums of
  // a quad add in sg order.
  constexpr int NQ = G * D / 4;
  const int nsg = nthreads / NQ, q4 = tid % NQ, sg = tid / NQ, g = 4 * q4 / D;
  const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(a.ws_o + (s0 * a.n_kv + h) * G * D), (short)0, 0x7fffffff, 0x00020000);
  const int stride_b = a.n_kv * G * D * 4;  // bytes from one split to the next
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int sp0 = sg; sp0 < nsplit; sp0 += 8 * nsg) {
    float4 x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int sp = sp0 + i * nsg;
      typedef float f4v __attribute__((ext_vector_type(4)));
      const f4v v = __builtin_bit_cast(
          f4v, __builtin_amdgcn_raw_buffer_load_b128(ro, (sp < nsplit ? sp : 0) * stride_b + 16 * q4, 0, 16));
      x[i] = make_float4(v.x, v.y, v.z, v.w);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int sp = sp0 + i * nsg;
      if (sp < nsplit) O = axpy4(s_wt[sp * G + g], x[i], O);
    }
  }
  float4 *s_part = reinterpret_cast<float4 *>(s_wt + kMaxSplits * G);
  s_part[tid] = O;
  __syncthreads();
  if (tid < NQ) {
    float4 T = s_part[tid];
    for (int k = 1; k < nsg; ++k) {
      const float4 y = s_part[k * NQ + tid];
      T.x += y.x;
      T.y += y.y;
      T.z += y.z;
      T.w += y.w;
    }
    const float Ls = s_L[g];
    st4(a.out + b * a.out_bstride + (long long)h * G * D + 4 * tid,
        make_float4(T.x / Ls, T.y / Ls, T.z / Ls, T.w / Ls));
  }
}

// ---------------------------------------------------------------------------
// Split-K decode attention with a reference merge, head_dim 128.
//
// Reference merge.  Softmax is invariant to the value subtracted before the
// exponential, so every split of a (sequence, kv head) weighs its rows by
// exp2(s - R[g]), where R[g] is the score of row `position` (the newest row)
// for q head g.  Every workgroup loads that one key row (the raw new key
// when the append is fused, rotated with the same table entry) and computes
// R[g] with the same instructions as the row's own score, so all splits use
// identical references and their unnormalised sums simply add:
//   out[g] = (sum over splits of O_s[g]) / (sum over splits of l_s[g]).
// The splits add O_s and l_s into acc with device-scope float atomics (2 KB
// per split); the last workgroup of the (sequence, kv head), found with a
// ticket, divides and clears acc for the next launch: the merge loads 2 KB
// in one round trip instead of every split's partial state, and the
// per-row-group maxima, weights and rescales of a running-maximum softmax
// disappear.  The newest row's own weight is exp2(0) = 1, so the sum of
// weights is at least 1 and cannot underflow.
//
// Exact path.  A split whose largest score exceeds R by more than kRefSlack
// (its weights could overflow) -- or that meets a non-finite score --
// recomputes its rows with a running maximum per row group, stores that
// partial state and flags itself in a mask; the merging workgroup folds
// flagged splits into the reference sums.
//
// Rows.  Workgroup = W waves = 4W row groups of 16 lanes.  Lane j of a row
// group holds dims {4j..4j+3} and {64+4j..64+4j+3} of a row: a dot product
// is a DPP row sum, and the RoPE pair (i, i+64) of a q/k element sits in one
// lane.  Row group r takes rows t0 + p*4W*RPG + i*4W + r (pass p, i < RPG);
// the loads of a pass -- and, for the first pass, of q, the table entry, the
// reference key and the new value -- are issued as one batch.  The 4W
// row-group states add through LDS (one reference: plain sums).
//
// Summation order across splits follows the order of the atomics, so the
// last bits of an output can differ between runs (the two older merges of
// decode_kernel are deterministic).
// ---------------------------------------------------------------------------
// Phase stamps of a measurement build (BNR_TIMELINE): wave 0 reads
// the 100 MHz real-time counter at the ends of the phases and thread 0
// stores them when the workgroup ends.  Scheduling barriers keep each read
// between the instructions of the phases it separates.
#if defined(BNR_TIMELINE)
#define BNR_STAMP(k)                                   \
  do {                                                 \
    __builtin_amdgcn_sched_barrier(0);                 \
    stamp[k] = __builtin_amdgcn_s_memrealtime();       \
    __builtin_amdgcn_sched_barrier(0);                 \
  } while (0)
#else
#define BNR_STAMP(k) ((void)0)
#endif

template <int G, int W, int RPG, bool RAGGED>
__global__ __launch_bounds__(64 * W) void decode_reg_kernel(DecodeArgs a) {
#if defined(BNR_TIMELINE)
  unsigned long long stamp[kTimelineStamps] = {};
  stamp[0] = __builtin_amdgcn_s_memrealtime();
  auto flush_stamps = [&]() {
    if (threadIdx.x == 0 && a.timeline) {
      const long long wg = blockIdx.x + (long long)gridDim.x * (blockIdx.y + (long long)gridDim.y * blockIdx.z);
      for (int k = 0; k < kTimelineStamps; ++k) a.timeline[wg * kTimelineStamps + k] = stamp[k];
    }
  };
#else
  auto flush_stamps = []() {};
#endif
  constexpr int D = kHeadDim;
  constexpr int NRG = 4 * W;  // row groups
  static_assert(G * D <= kAccL && G <= 4, "accumulator layout holds up to 4 q heads");
  static_assert(3 * kMaxSplits * G + 4 * 64 * W <= NRG * G * D,
                "s_o holds the deterministic merge's (m, l), weights and partial sums");
  __shared__ __attribute__((aligned(16))) float s_o[NRG][G][D];
  __shared__ float s_m[NRG][G], s_l[NRG][G], s_w[NRG][G], s_M[G], s_L[G], s_R[G];
  __shared__ unsigned long long s_mk[4];
  __shared__ int s_last, s_over[W];

  const int tid = threadIdx.x;
  const int rg = tid >> 4;
  const int j = tid & 15;
  const int b = blockIdx.z;
  const int s = blockIdx.x;
  const int nsplit = a.split_off[b + 1] - a.split_off[b];
  if (RAGGED && s >= nsplit) {
    flush_stamps();
    return;
  }
  const int h = blockIdx.y;
  const int pos = a.positions[b];
  const int L = pos + 1;
  const int t0 = s * a.rows_per_split;
  const int t1 = min(t0 + a.rows_per_split, L);

  float *kc = a.k_cache + b * a.cache_bstride + h * a.kv_stride;
  float *vc = a.v_cache + b * a.cache_bstride + h * a.kv_stride;

  // ---- loads, in use order: q (+cos/sin), the reference key row, the new
  // value (owner of `position` only), the first pass's K and V rows.
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
  const bool fused = a.k_new != nullptr;
  const float *kref = fused ? a.k_new + b * a.kn_bstride + h * D : kc + (long long)pos * D;
  float4 rklo = ld4(kref + 4 * j), rkhi = ld4(kref + 64 + 4 * j);
  const bool own_pos = fused && pos >= t0 && pos < t1;
  float4 nvlo = make_float4(0.f, 0.f, 0.f, 0.f), nvhi = nvlo;
  if (own_pos) {
    const float *vn = a.v_new + b * a.kn_bstride + h * D;
    nvlo = ld4(vn + 4 * j);
    nvhi = ld4(vn + 64 + 4 * j);
  }
  float4 klo[RPG], khi[RPG], vlo[RPG], vhi[RPG];
  bool valid[RPG];
  auto load_pass = [&](int tp) {
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int t = tp + i * NRG + rg;
      valid[i] = t < t1;
      const long long off = (long long)(valid[i] ? t : t0) * D;
      klo[i] = ld4_nt(kc + off + 4 * j);
      khi[i] = ld4_nt(kc + off + 64 + 4 * j);
    }
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const long long off = (long long)(valid[i] ? tp + i * NRG + rg : t0) * D;
      vlo[i] = ld4_nt(vc + off + 4 * j);
      vhi[i] = ld4_nt(vc + off + 64 + 4 * j);
    }
  };
  load_pass(t0);
  __builtin_amdgcn_sched_barrier(0);  // keep every load of the batch ahead of the math
  BNR_STAMP(1);

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
  if (fused && rope) {
    rot4(rklo, rkhi, cs, sn, rklo, rkhi);
    if (a.k_rot && s == 0 && rg == 0) {
      float *kr = a.k_rot + b * a.kn_bstride + h * D;
      st4(kr + 4 * j, rklo);
      st4(kr + 64 + 4 * j, rkhi);
    }
  }
  // Reference scores: exactly the score row `position` gets below.
  float R[G];
#pragma unroll
  for (int g = 0; g < G; ++g) R[g] = row_sum16(dot8(qlo[g], qhi[g], rklo, rkhi));

  // The owner of `position` substitutes the new row -- also where a masked
  // row past the split's end was clamped onto it: that cache row is not
  // written yet, and its stale contents would turn the zero weight into
  // 0 * inf = NaN -- and appends the row.
  auto put_new = [&](int tp, bool store) {
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int t = tp + i * NRG + rg;
      if ((valid[i] ? t : t0) == pos) {
        klo[i] = rklo;
        khi[i] = rkhi;
        vlo[i] = nvlo;
        vhi[i] = nvhi;
        if (store && valid[i]) {
          st4(kc + (long long)pos * D + 4 * j, rklo);
          st4(kc + (long long)pos * D + 64 + 4 * j, rkhi);
          st4(vc + (long long)pos * D + 4 * j, nvlo);
          st4(vc + (long long)pos * D + 64 + 4 * j, nvhi);
        }
      }
    }
  };

  // ---- rows weighed against the reference ----
  float l[G], mx[G];
  float4 olo[G], ohi[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    l[g] = 0.f;
    mx[g] = -INFINITY;
    olo[g] = make_float4(0.f, 0.f, 0.f, 0.f);
    ohi[g] = olo[g];
  }
  for (int tp = t0; tp < t1; tp += NRG * RPG) {
    if (tp > t0) load_pass(tp);
    if (own_pos) put_new(tp, true);
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = row_sum16(dot8(qlo[g], qhi[g], klo[i], khi[i]));
        const float sc = valid[i] ? d : -INFINITY;
        mx[g] = fmaxf(mx[g], sc);
        const float pr = fast_exp2(sc - R[g]);
        l[g] += pr;
        olo[g] = axpy4(pr, vlo[i], olo[g]);
        ohi[g] = axpy4(pr, vhi[i], ohi[g]);
      }
    }
  }
  BNR_STAMP(2);
  // ---- the row groups add through LDS (fast path) ----
  // Written before the barrier that decides the path (one barrier fewer):
  // the exact path discards these sums and rewrites s_o after it.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    st4(&s_o[rg][g][4 * j], olo[g]);
    st4(&s_o[rg][g][64 + 4 * j], ohi[g]);
    if (j == 0) s_l[rg][g] = l[g];
  }
  int over = 0;
#pragma unroll
  for (int g = 0; g < G; ++g)
    over |= !(mx[g] <= R[g] + kRefSlack) | !(R[g] > -INFINITY && R[g] < INFINITY);
  // One barrier decides the path: each wave posts whether any of its lanes
  // needs the exact path (every wave writes its slot, so nothing is cleared).
  const bool wave_over = __ballot(over) != 0;  // every lane votes
  if ((tid & 63) == 0) s_over[tid >> 6] = wave_over;
  __syncthreads();
  BNR_STAMP(3);
  bool exact = false;
#pragma unroll
  for (int w = 0; w < W; ++w) exact |= s_over[w] != 0;

  // Host-slice calls: the output of (sequence b, kv head h) is in host
  // memory -- every thread's stores complete, then one release store tells
  // the waiting host thread.
  auto signal = [&]() {
    if (a.done) signal_host(a.done + b * a.n_kv + h, a.seq);
  };
  const int gs = a.split_off[b] + s;  // global split index
  const bool det = a.merge_det != 0;
  float *acc = a.acc + ((long long)b * a.n_kv + h) * kAccStride;
  if (!exact) {
    for (int e = tid; e < G * D; e += 64 * W) {
      const int g = e / D, dim = e % D;
      float O = s_o[0][g][dim];
#pragma unroll
      for (int r = 1; r < NRG; ++r) O += s_o[r][g][dim];
      if (nsplit == 1) {
        float Ls = s_l[0][g];
#pragma unroll
        for (int r = 1; r < NRG; ++r) Ls += s_l[r][g];
        a.out[b * a.out_bstride + (long long)h * G * D + e] = O / Ls;
      } else if (det) {
        st_agent(&a.ws_o[((long long)gs * a.n_kv + h) * G * D + e], O);
      } else {
        add_agent(acc + e, O);
      }
    }
    if (nsplit == 1) {
      signal();
      flush_stamps();
      return;
    }
    if (tid < G) {
      float Ls = s_l[0][tid];
#pragma unroll
      for (int r = 1; r < NRG; ++r) Ls += s_l[r][tid];
      if (det) {
        float *ml = reinterpret_cast<float *>(&a.ws_ml[((long long)gs * a.n_kv + h) * G + tid]);
        st_agent(ml, R[tid]);
        st_agent(ml + 1, Ls);
      } else {
        add_agent(acc + kAccL + tid, Ls);
      }
    }
  } else {
    // ---- exact path: the rows again, a running maximum per row group ----
    float m_run[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m_run[g] = -INFINITY;
      l[g] = 0.f;
      olo[g] = make_float4(0.f, 0.f, 0.f, 0.f);
      ohi[g] = olo[g];
    }
    for (int tp = t0; tp < t1; tp += NRG * RPG) {
      load_pass(tp);
      if (own_pos) put_new(tp, false);
#pragma unroll
      for (int i = 0; i < RPG; ++i) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float d = row_sum16(dot8(qlo[g], qhi[g], klo[i], khi[i]));
          const float sc = valid[i] ? d : -INFINITY;
          const float m_new = fmaxf(m_run[g], sc);
          if (m_new == -INFINITY) continue;  // no valid row yet in this row group
          const float alpha = fast_exp2(m_run[g] - m_new), pr = fast_exp2(sc - m_new);
          l[g] = fmaf(l[g], alpha, pr);
          olo[g] = axpy4(pr, vlo[i], scale4(alpha, olo[g]));
          ohi[g] = axpy4(pr, vhi[i], scale4(alpha, ohi[g]));
          m_run[g] = m_new;
        }
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      st4(&s_o[rg][g][4 * j], olo[g]);
      st4(&s_o[rg][g][64 + 4 * j], ohi[g]);
      if (j == 0) {
        s_m[rg][g] = m_run[g];
        s_l[rg][g] = l[g];
      }
    }
    __syncthreads();
    if (tid < G) {
      float M = -INFINITY;
      for (int r = 0; r < NRG; ++r) M = fmaxf(M, s_m[r][tid]);
      float Ls = 0.f;
      for (int r = 0; r < NRG; ++r) {
        const float wr = M == -INFINITY ? 0.f : fast_exp2(s_m[r][tid] - M);
        s_w[r][tid] = wr;
        Ls = fmaf(s_l[r][tid], wr, Ls);
      }
      s_M[tid] = M;
      s_L[tid] = Ls;
    }
    __syncthreads();
    for (int e = tid; e < G * D; e += 64 * W) {
      const int g = e / D, dim = e % D;
      float O = 0.f;
      for (int r = 0; r < NRG; ++r) O = fmaf(s_w[r][g], s_o[r][g][dim], O);
      if (nsplit == 1)
        a.out[b * a.out_bstride + (long long)h * G * D + e] = O / s_L[g];
      else
        st_agent(&a.ws_o[((long long)gs * a.n_kv + h) * G * D + e], O);
    }
    if (nsplit == 1) {
      signal();
      flush_stamps();
      return;
    }
    if (tid < G) {
      float *ml = reinterpret_cast<float *>(&a.ws_ml[((long long)gs * a.n_kv + h) * G + tid]);
      st_agent(ml, s_M[tid]);
      st_agent(ml + 1, s_L[tid]);
    }
    if (tid == 0 && !det) {
      unsigned long long *mask = reinterpret_cast<unsigned long long *>(acc + kAccMask) + (s >> 6);
      (void)__hip_atomic_fetch_or(mask, 1ull << (s & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // ---- ticket: the last workgroup of this (sequence, kv head) divides ----
  // Every wave's device-scope adds and partial stores have completed before
  // the ticket is taken; the merging workgroup reads them with atomic
  // read-modify-writes (ref_merge).
  BNR_STAMP(4);
  __builtin_amdgcn_s_waitcnt(0);
  BNR_STAMP(5);
  if (tid < G) s_R[tid] = R[tid];
  __syncthreads();
  // Host-slice calls: split 0's rotated q and k (in host memory) reach the
  // host before its ticket, hence before the merging workgroup's completion
  // word (a system-scope release: this XCD's L2 is written back).
  if (a.done && s == 0 && tid == 0 && (a.q_rot || a.k_rot))
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
  unsigned *ctr = a.counters + (b * a.n_kv + h) * kCounterStride;
  if (tid == 0) {
    const unsigned ticket =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (ticket == (unsigned)(nsplit - 1));
  }
  __syncthreads();
  BNR_STAMP(6);
  if (!s_last) {
    flush_stamps();
    return;
  }
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (det) {
    // s_o is free now: it holds the splits' (m, l) and weights
    float2 *s_ml = reinterpret_cast<float2 *>(&s_o[0][0][0]);
    det_merge<G>(a, b, h, nsplit, s_ml, reinterpret_cast<float *>(s_ml + kMaxSplits * G), s_L, tid,
                 64 * W);
  } else {
    ref_merge<G>(a, b, h, acc, s_R, s_L, s_mk, tid, 64 * W);
  }
  signal();
#if defined(BNR_TIMELINE)
  __builtin_amdgcn_s_waitcnt(0);  // the output stores have completed
  BNR_STAMP(7);
#endif
  flush_stamps();
}

template <int G, int W, bool RAGGED>
hipError_t launch_reg_wr(const DecodeArgs &a, hipStream_t s) {
  dim3 grid(a.max_splits, a.n_kv, a.batch), block(64 * W);
  switch (a.rpg) {
    case 1: decode_reg_kernel<G, W, 1, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 2: decode_reg_kernel<G, W, 2, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 3: decode_reg_kernel<G, W, 3, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 4: decode_reg_kernel<G, W, 4, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 5: decode_reg_kernel<G, W, 5, RAGGED><<<grid, block, 0, s>>>(a); break;
    case 6: decode_reg_kernel<G, W, 6, RAGGED><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

#if defined(BNR_TIMELINE)
// Measurement builds only.  One lane runs n dependent device-scope
// operations (each address depends on the previous result, or an
// s_waitcnt separates them) and stores the elapsed 100 MHz ticks: the round
// trip of the operations the decode's merge chain is made of.  mode 0:
// fetch_add with return (the ticket); 1: add without return, then wait for
// it (the sums); 2: exchange (the merging read); 3: agent-scope load.
__global__ void rt_probe_kernel(unsigned *buf, int n, int mode, unsigned long long *out) {
  if (threadIdx.x != 0) return;
  unsigned v = 1;
  const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
  for (int i = 0; i < n; ++i) {
    unsigned *p = buf + 64 * (v & 1);
    if (mode == 0) {
      v += __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (mode == 1) {
      (void)__hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      v += 2;
    } else if (mode == 2) {
      v += __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      v += __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
  out[0] = t1 - t0;
  out[1] = v;
}

// Launches that do (almost) nothing: the graph's launch-to-launch cost of
// a grid, bare, with the decode's argument block (one value read from it),
// with a 64 KB LDS allocation (one word written and read), or both.
__global__ void empty_kernel() {}
__global__ void empty_args_kernel(DecodeArgs a) {
  if (threadIdx.x == 0 && a.seq == 0x7fffffffu) a.counters[0] = 0;  // never true
}
__global__ __launch_bounds__(512) void empty_lds_kernel(unsigned flag) {
  __shared__ float s_big[16384];
  s_big[threadIdx.x * 32] = (float)threadIdx.x;
  __syncthreads();
  if (s_big[(threadIdx.x * 37) & 16383] == -1.f && flag == 0x7fffffffu) s_big[0] = 1.f;
}
// ... or one word per workgroup written to buf: mode 4 a plain store, 5 a
// non-temporal store, 6 a device-scope atomic add, 7 a system-scope store.
__global__ void empty_write_kernel(unsigned *buf, int mode) {
  if (threadIdx.x != 0) return;
  unsigned *p = buf + 64 * (blockIdx.x & 255);
  if (mode == 4) *p = blockIdx.x;
  else if (mode == 5) __builtin_nontemporal_store((unsigned)blockIdx.x, p);
  else if (mode == 6) (void)__hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  else __hip_atomic_store(p, (unsigned)blockIdx.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__global__ __launch_bounds__(512) void empty_args_lds_kernel(DecodeArgs a) {
  __shared__ float s_big[16384];
  s_big[threadIdx.x * 32] = (float)threadIdx.x;
  __syncthreads();
  if (s_big[(threadIdx.x * 37) & 16383] == -1.f && a.seq == 0x7fffffffu) a.counters[0] = 0;
}
// ... and with 160 VGPRs allocated, as the 8-wave decode kernel has.
__global__ __launch_bounds__(512) void empty_full_kernel(DecodeArgs a) {
  __shared__ float s_big[16384];
  asm volatile("v_mov_b32 v159, 0" ::: "v159");
  s_big[threadIdx.x * 32] = (float)threadIdx.x;
  __syncthreads();
  if (s_big[(threadIdx.x * 37) & 16383] == -1.f && a.seq == 0x7fffffffu) a.counters[0] = 0;
}
#endif

}  // namespace

#if defined(BNR_TIMELINE)
hipError_t launch_rt_probe(unsigned *buf, int n, int mode, unsigned long long *out, hipStream_t s) {
  rt_probe_kernel<<<1, 64, 0, s>>>(buf, n, mode, out);
  return hipGetLastError();
}
hipError_t launch_empty(int wgs, int threads, int mode, unsigned *buf, hipStream_t s) {
  DecodeArgs a{};
  if (mode >= 4 && mode <= 7) empty_write_kernel<<<wgs, threads, 0, s>>>(buf, mode);
  else if (mode == 0) empty_kernel<<<wgs, threads, 0, s>>>();
  else if (mode == 1) empty_args_kernel<<<wgs, threads, 0, s>>>(a);
  else if (mode == 2) empty_lds_kernel<<<wgs, threads, 0, s>>>(0u);
  else if (mode == 3) empty_args_lds_kernel<<<wgs, threads, 0, s>>>(a);
  else empty_full_kernel<<<wgs, threads, 0, s>>>(a);
  return hipGetLastError();
}
#endif

hipError_t launch_decode_ref(const DecodeArgs &a, hipStream_t s) {
  if (!a.acc) return hipErrorInvalidValue;
  bool ragged = false;
  for (int b = 0; b < a.batch; ++b)
    ragged |= (a.split_off[b + 1] - a.split_off[b]) != a.max_splits;
  if (a.ref_waves == 8) {
    switch (a.group) {
      case 1: return ragged ? launch_reg_wr<1, 8, true>(a, s) : launch_reg_wr<1, 8, false>(a, s);
      case 2: return ragged ? launch_reg_wr<2, 8, true>(a, s) : launch_reg_wr<2, 8, false>(a, s);
      case 4: return ragged ? launch_reg_wr<4, 8, true>(a, s) : launch_reg_wr<4, 8, false>(a, s);
      default: return hipErrorInvalidValue;
    }
  }
  switch (a.group) {
    case 1: return ragged ? launch_reg_wr<1, 4, true>(a, s) : launch_reg_wr<1, 4, false>(a, s);
    case 2: return ragged ? launch_reg_wr<2, 4, true>(a, s) : launch_reg_wr<2, 4, false>(a, s);
    case 4: return ragged ? launch_reg_wr<4, 4, true>(a, s) : launch_reg_wr<4, 4, false>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bnr
