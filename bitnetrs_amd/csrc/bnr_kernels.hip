// bnr_kernels.hip -- gfx950 kernels of the GQA attention hot path.
//
//  rope_append_kernel  half-split RoPE of q/k + head-major KV append
//  decode_kernel<G,RPG> split-K decode attention, head_dim 128, optional
//                       fused RoPE + append, last-workgroup merge
//  decode_generic_kernel any head_dim / group size
//
// Wave64 throughout.  The decode kernel reads each K/V row of a kv head once
// and serves the G query heads of the group from registers (the reference
// re-reads every row once per query head, bitnet-cpu/src/attention.rs:
// 170-204).
#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

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

// ---------------------------------------------------------------------------
// Split-K decode attention, head_dim 128.
//
// Workgroup = 256 lanes = 16 row groups of 16 lanes.  Lane j of a row group
// holds dims {4j..4j+3} and {64+4j..64+4j+3} of a row: one float4 from each
// half, so one instruction of a wave reads four 256-byte row halves, and the
// half-split RoPE pair (i, i+64) of a q/k element sits in the same lane.
//
// Row r of pass p, iteration i of row group rg is t0 + p*16*RPG + i*16 + rg.
// Each row group keeps an online-softmax state (m, l, o[G][8 dims per lane]);
// the 16 states are merged through LDS into one (m, l, o) per workgroup,
// written to the split workspace, and the last workgroup of a
// (sequence, kv head) to arrive -- found with an agent-scope ticket -- merges
// all splits and writes the output.  The ticket counter is reset by that
// workgroup, so no memset is needed between launches.
// ---------------------------------------------------------------------------
template <int G, int RPG>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
  constexpr int D = kHeadDim;
  __shared__ float s_o[16][G][D];
  __shared__ float s_m[16][G];
  __shared__ float s_l[16][G];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int rg = tid >> 4;
  const int j = tid & 15;

  // blockIdx.x -> (sequence b, split s); the table is in kernel arguments.
  int b = 0;
  while ((int)blockIdx.x >= a.split_off[b + 1]) ++b;
  const int s = (int)blockIdx.x - a.split_off[b];
  const int nsplit = a.split_off[b + 1] - a.split_off[b];
  const int h = blockIdx.y;
  const int pos = a.positions[b];
  const int L = pos + 1;
  const int t0 = s * a.rows_per_split;
  const int t1 = min(t0 + a.rows_per_split, L);

  float *kc = a.k_cache + b * a.cache_bstride + h * a.kv_stride;
  float *vc = a.v_cache + b * a.cache_bstride + h * a.kv_stride;
  const float *qb = a.q + b * a.q_bstride + (long long)h * G * D;

  // ---- q for the G heads of this kv head (rotated here when fused) ----
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

  // ---- the new token's rotated key and value (fused append) ----
  const bool fused = a.k_new != nullptr;
  float4 nklo = make_float4(0.f, 0.f, 0.f, 0.f), nkhi = nklo, nvlo = nklo, nvhi = nklo;
  const bool own_pos = fused && pos >= t0 && pos < t1;
  if (fused && (own_pos || (a.k_rot && s == 0))) {
    const float *kn = a.k_new + b * a.kn_bstride + h * D;
    const float *vn = a.v_new + b * a.kn_bstride + h * D;
    rot4(ld4(kn + 4 * j), ld4(kn + 64 + 4 * j), cs, sn, nklo, nkhi);
    nvlo = ld4(vn + 4 * j);
    nvhi = ld4(vn + 64 + 4 * j);
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
    float4 klo[RPG], khi[RPG], vlo[RPG], vhi[RPG];
    bool valid[RPG];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      const int t = tp + i * 16 + rg;
      valid[i] = t < t1;
      const long long off = (long long)(valid[i] ? t : t0) * D;
      klo[i] = ld4(kc + off + 4 * j);
      khi[i] = ld4(kc + off + 64 + 4 * j);
      vlo[i] = ld4(vc + off + 4 * j);
      vhi[i] = ld4(vc + off + 64 + 4 * j);
    }
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
    float sc[RPG][G];
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float d = row_sum16(dot8(qlo[g], qhi[g], klo[i], khi[i]));
        sc[i][g] = valid[i] ? d : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float mp = sc[0][g];
#pragma unroll
      for (int i = 1; i < RPG; ++i) mp = fmaxf(mp, sc[i][g]);
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
  }

  // ---- merge the 16 row-group states through LDS ----
#pragma unroll
  for (int g = 0; g < G; ++g) {
    st4(&s_o[rg][g][4 * j], olo[g]);
    st4(&s_o[rg][g][64 + 4 * j], ohi[g]);
    if (j == 0) {
      s_m[rg][g] = m_run[g];
      s_l[rg][g] = l_run[g];
    }
  }
  __syncthreads();

  const int gs = a.split_off[b] + s;  // global split index
  for (int e = tid; e < G * D; e += 256) {
    const int g = e / D, dim = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) M = fmaxf(M, s_m[r][g]);
    float Ls = 0.f, O = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float w = fast_exp2(s_m[r][g] - M);  // 0 for an empty row group
      Ls = fmaf(s_l[r][g], w, Ls);
      O = fmaf(s_o[r][g][dim], w, O);
    }
    if (nsplit == 1) {
      a.out[b * a.out_bstride + ((long long)h * G + g) * D + dim] = O / Ls;
    } else {
      a.ws_o[(((long long)gs * a.n_kv + h) * G + g) * D + dim] = O;
      if (dim == 0) a.ws_ml[((long long)gs * a.n_kv + h) * G + g] = make_float2(M, Ls);
    }
  }
  if (nsplit == 1) return;

  // ---- last workgroup of this (sequence, kv head) merges the splits ----
  __threadfence();
  __syncthreads();
  unsigned *ctr = a.counters + b * a.n_kv + h;
  if (tid == 0) {
    const unsigned ticket =
        __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (ticket == (unsigned)(nsplit - 1));
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // (max, sum) of every split of this kv head into LDS (reusing s_o).
  float2 *s_ml = reinterpret_cast<float2 *>(&s_o[0][0][0]);
  const int gs0 = a.split_off[b];
  for (int idx = tid; idx < nsplit * G; idx += 256) {
    const int sp = idx / G, g = idx % G;
    s_ml[idx] = a.ws_ml[((long long)(gs0 + sp) * a.n_kv + h) * G + g];
  }
  __syncthreads();
  for (int e = tid; e < G * D; e += 256) {
    const int g = e / D, dim = e % D;
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, s_ml[sp * G + g].x);
    float Ls = 0.f, O = 0.f;
    const float *po = a.ws_o + (((long long)gs0 * a.n_kv + h) * G + g) * D + dim;
    const long long step = (long long)a.n_kv * G * D;
    int sp = 0;
    for (; sp + 8 <= nsplit; sp += 8) {
      float ov[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) ov[u] = po[(sp + u) * step];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float2 ml = s_ml[(sp + u) * G + g];
        const float w = fast_exp2(ml.x - M);
        Ls = fmaf(ml.y, w, Ls);
        O = fmaf(ov[u], w, O);
      }
    }
    for (; sp < nsplit; ++sp) {
      const float2 ml = s_ml[sp * G + g];
      const float w = fast_exp2(ml.x - M);
      Ls = fmaf(ml.y, w, Ls);
      O = fmaf(po[sp * step], w, O);
    }
    a.out[b * a.out_bstride + ((long long)h * G + g) * D + dim] = O / Ls;
  }
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

template <int G>
hipError_t launch_decode_g(const DecodeArgs &a, hipStream_t s) {
  dim3 grid(a.split_off[a.batch], a.n_kv), block(256);
  switch (a.rpg) {
    case 1: decode_kernel<G, 1><<<grid, block, 0, s>>>(a); break;
    case 2: decode_kernel<G, 2><<<grid, block, 0, s>>>(a); break;
    case 4: decode_kernel<G, 4><<<grid, block, 0, s>>>(a); break;
    case 8: decode_kernel<G, 8><<<grid, block, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_append(const RopeAppendArgs &a, hipStream_t s) {
  const long long total = (long long)a.n_tokens * (a.n_heads + 2 * a.n_kv) * (a.head_dim / 2);
  if (total == 0) return hipSuccess;
  long long blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
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

hipError_t launch_decode_generic(const DecodeGenericArgs &a, hipStream_t s) {
  decode_generic_kernel<<<dim3(a.n_heads), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace bnr
