// bnr_gemv.hip -- W2A8 ternary GEMV for gfx950 (Backend::ternary_gemv_preq).
//
// out[i] = (float)(sum_j W[i][j] * a[j]) * scale, with W in {-1, 0, +1}
// stored 2 bits per weight (row-aligned, ceil(K/4) bytes per row; code
// 0b00 -> +1, 0b01 -> 0, 0b10 -> -1, 0b11 -> 0, weight 4b+p at bits 2p of
// byte b) and a[] int8.  The integer sum is exact, so the result is
// bit-identical to the reference's (bitnet-cpu/src/gemv.rs:251-310).
//
// Memory-bound: each packed weight byte is read once.  A workgroup owns 16
// rows, 16 lanes per row; a lane takes the row's 16-byte pieces j, j+16, ...
// (64 weights each).  The K activations are staged in LDS once per workgroup
// and pass (4096 per pass), transposed so that one v_dot4_i32_i8 pairs four
// decoded weights with their activations without unpacking the 2-bit codes
// into bytes.
#include "bnr_internal.h"

#include <hip/hip_runtime.h>

namespace bnr {
namespace {

// 16 bytes with the non-temporal hint (global_load_dwordx4 ... nt), for
// weights: a decode token streams every matrix once (524 MB of ternary
// weights and 328 MB of LM head per token, more than the 256 MB MALL).
// Measured on MI355X: the 2B decode token 1.112 -> 1.069 ms, the
// 128256 x 2560 LM head 62.7-64.2 -> 57.9-58.8 us.
__device__ __forceinline__ uint4 ld16_nt(const void *p) {
  typedef unsigned u4v __attribute__((ext_vector_type(4)));
  const u4v v = __builtin_nontemporal_load(reinterpret_cast<const u4v *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

constexpr int kRowsPerWg = 16;
constexpr int kPass = 4096;                 // activations per LDS pass
constexpr int kGroups = kPass / 16;         // 16-activation groups per pass
constexpr int kPieces = kPass / 64;         // 16-byte weight pieces per row and pass
constexpr int kPiecesPerLane = kPieces / 16;

// Decode table for v_perm_b32: byte c of kCodeValue is the int8 value of
// code c (+1, 0, -1, 0).
constexpr unsigned kCodeValue = 0x00FF0001u;

// One packed dword w = weights 16g .. 16g+15 (weight 16g + 4k + p at bits
// 8k + 2p).  (w >> 2p) & 0x03030303 puts the codes of weights 4k + p,
// k = 0..3, in its four bytes; v_perm maps each code to its value.  act.{x,y,z,w}
// hold the activations of the same positions for p = 0, 1, 2, 3.
__device__ __forceinline__ int dot16(unsigned w, uint4 act, int acc) {
  const unsigned m = 0x03030303u;
  acc = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(0u, kCodeValue, w & m), (int)act.x, acc, false);
  acc = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(0u, kCodeValue, (w >> 2) & m), (int)act.y, acc, false);
  acc = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(0u, kCodeValue, (w >> 4) & m), (int)act.z, acc, false);
  acc = __builtin_amdgcn_sdot4((int)__builtin_amdgcn_perm(0u, kCodeValue, (w >> 6) & m), (int)act.w, acc, false);
  return acc;
}

// 16 activations x0..x3 (dword t = activations 4t .. 4t+3) -> the four
// dwords dot16 expects: dword p = activations p, 4+p, 8+p, 12+p (a 4x4 byte
// transpose).
__device__ __forceinline__ uint4 transpose_bytes(uint4 x) {
  const unsigned t0 = __builtin_amdgcn_perm(x.y, x.x, 0x05010400u);  // x0b0 x1b0 x0b1 x1b1
  const unsigned t1 = __builtin_amdgcn_perm(x.y, x.x, 0x07030602u);  // x0b2 x1b2 x0b3 x1b3
  const unsigned t2 = __builtin_amdgcn_perm(x.w, x.z, 0x05010400u);  // x2b0 x3b0 x2b1 x3b1
  const unsigned t3 = __builtin_amdgcn_perm(x.w, x.z, 0x07030602u);  // x2b2 x3b2 x2b3 x3b3
  return make_uint4(__builtin_amdgcn_perm(t2, t0, 0x05040100u), __builtin_amdgcn_perm(t2, t0, 0x07060302u),
                    __builtin_amdgcn_perm(t3, t1, 0x05040100u), __builtin_amdgcn_perm(t3, t1, 0x07060302u));
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lanef(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Sum over the 16 lanes of a DPP row.
__device__ __forceinline__ int row_sum16_i(int v) {
  v += dpp_i<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_i<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_i<0x141>(v);  // row_half_mirror
  v += dpp_i<0x140>(v);  // row_mirror
  return v;
}
// Sum over aligned groups of L = 4, 8 or 16 lanes, in the group's first lane.
template <int L>
__device__ __forceinline__ int lane_group_sum_i(int v) {
  v += dpp_i<0xB1>(v);
  v += dpp_i<0x4E>(v);
  if (L >= 8) v += dpp_i<0x141>(v);
  if (L >= 16) v += dpp_i<0x140>(v);
  return v;
}

// Bytes [off, off+16) of p, the ones at or past `limit` read as zero.
__device__ __forceinline__ uint4 load16_bounded(const uint8_t *p, long long off, long long limit) {
  unsigned d[4] = {0u, 0u, 0u, 0u};
  for (int b = 0; b < 16; ++b)
    if (off + b < limit) d[b >> 2] |= (unsigned)p[off + b] << (8 * (b & 3));
  return make_uint4(d[0], d[1], d[2], d[3]);
}

// Rows [16*wg, 16*wg+16) of one matrix: out[row] = (float)dot * scale.
// VEC: rows start 16-byte aligned with a whole number of 16-byte pieces
// (ceil(K/4) % 16 == 0) and the activations are 16-byte aligned.
template <bool VEC>
__device__ __forceinline__ void gemv_rows(const uint8_t *w, const int8_t *act, float *out,
                                          int out_features, int in_features,
                                          long long packed_cols, float scale, int wg,
                                          uint4 *s_act) {
  const int tid = threadIdx.x, slot = tid >> 4, j = tid & 15;
  const int row = wg * kRowsPerWg + slot;
  const long long prow = (long long)min(row, out_features - 1) * packed_cols;
  int acc = 0;
  for (int k0 = 0; k0 < in_features; k0 += kPass) {
    const int kn = min(kPass, in_features - k0);     // activations of this pass
    const long long b0 = prow + k0 / 4;              // first packed byte of the pass
    const int nb = (kn + 3) / 4;                     // packed bytes of the pass
    // Activation groups first: loads return in order, so the small,
    // cache-resident activations arrive (and go to LDS) while the weights
    // are still in flight.
    uint4 xa[kGroups / 256];
#pragma unroll
    for (int t = 0; t < kGroups / 256; ++t) {
      const int a0 = 16 * (tid + 256 * t);
      if (VEC && a0 + 16 <= kn) {
        xa[t] = *reinterpret_cast<const uint4 *>(act + k0 + a0);
      } else {
        xa[t] = load16_bounded(reinterpret_cast<const uint8_t *>(act), (long long)k0 + a0,
                               (long long)k0 + kn);
      }
    }
    uint4 wv[kPiecesPerLane];
#pragma unroll
    for (int i = 0; i < kPiecesPerLane; ++i) {
      const int c = j + 16 * i;
      if (VEC) {
        wv[i] = 16 * c < nb ? ld16_nt(w + b0 + 16 * c) : make_uint4(0, 0, 0, 0);
      } else {
        wv[i] = 16 * c < nb ? load16_bounded(w, b0 + 16 * c, b0 + nb) : make_uint4(0, 0, 0, 0);
      }
    }
    __syncthreads();  // the previous pass has finished reading s_act
#pragma unroll
    for (int t = 0; t < kGroups / 256; ++t) {
      const int g = tid + 256 * t;
      s_act[(g & 3) * kPieces + (g >> 2)] = transpose_bytes(xa[t]);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPiecesPerLane; ++i) {
      const int c = j + 16 * i;
      if (16 * c < nb) {
        acc = dot16(wv[i].x, s_act[c], acc);
        acc = dot16(wv[i].y, s_act[kPieces + c], acc);
        acc = dot16(wv[i].z, s_act[2 * kPieces + c], acc);
        acc = dot16(wv[i].w, s_act[3 * kPieces + c], acc);
      }
    }
  }
  acc = row_sum16_i(acc);
  if (j == 0 && row < out_features) out[row] = (float)acc * scale;
}

template <bool VEC>
__global__ __launch_bounds__(256) void ternary_gemv_kernel(TernaryGemvArgs a) {
  // Activations of the pass, transposed: group g (activations 16g..16g+15)
  // at s_act[(g % 4) * kPieces + g / 4], so that the 16 lanes of a row read
  // consecutive 16-byte slots.
  __shared__ uint4 s_act[kGroups];
  gemv_rows<VEC>(a.weight, a.act, a.out, a.out_features, a.in_features, a.packed_cols, a.scale,
                 blockIdx.x, s_act);
}

template <bool VEC>
__global__ __launch_bounds__(256) void ternary_gemv_group_kernel(TernaryGemvGroupArgs a) {
  __shared__ uint4 s_act[kGroups];
  const int b = blockIdx.x;
  // Matrix of this workgroup, selected with constant indices so that the
  // argument arrays stay in scalar registers.
  const uint8_t *w = a.weight[0];
  float *out = a.out[0];
  float scale = a.scale[0], ws = a.weight_scale[0];
  int m = a.out_features[0], off = 0;
#pragma unroll
  for (int i = 1; i < kMaxGemvGroup; ++i) {
    if (i < a.n && b >= a.wg_off[i]) {
      w = a.weight[i];
      out = a.out[i];
      scale = a.scale[i];
      ws = a.weight_scale[i];
      m = a.out_features[i];
      off = a.wg_off[i];
    }
  }
  if (a.act_absmax_dev) {
    // combined_scale = weight_scale * act_scale / 127.0 (gemv.rs:297), f32, left to right
    const float t = ws * *a.act_absmax_dev;
    scale = t / 127.0f;
  }
  gemv_rows<VEC>(w, a.act, out, m, a.in_features, a.packed_cols, scale, b - off, s_act);
}

// ---------------------------------------------------------------------------
// Ternary GEMV with the activation's RMSNorm and int8 quantisation as its
// prologue (the glue launch folded into the projection).  Every workgroup
// forms x from f32 inputs (a | a + b | max(a,0)^2 * b), reduces sum(x^2) and
// max|y| with the same tree, and so derives the same int8 activations and
// the same scale as norm_quant_kernel would; the int8 vector never leaves
// LDS.  The workgroup issues the (cache-resident) activation loads first and
// its weight loads right after, so the prologue runs under the weights'
// latency.  K <= 4096 NG (one LDS pass; NG = 1 or 2 16-activation groups
// per thread, the smallest that holds K: at K <= 4096 the kernel needs 74
// VGPRs and 6 workgroups fit a CU, with two groups 142 and 3);
// workgroup 0 writes h_out (mode residual), which must not alias a or b.
// A workgroup owns 256 / LPR rows, LPR lanes per row: every workgroup reads
// the whole of a (and b) and gamma, so a launch with many rows takes 32 or
// 64 rows per workgroup to read those vectors fewer times.
// ---------------------------------------------------------------------------
constexpr int kNormK = 8192;

// x from the glue inputs: a | a + b | max(a, 0)^2 * b (mode kGlue*).
__device__ __forceinline__ float norm_x_of(int mode, float u, float v) {
#pragma clang fp contract(off)
  if (mode == kGlueResidual) return u + v;
  if (mode == kGlueSqrelu) {
    const float r = fmaxf(u, 0.0f);
    return r * r * v;
  }
  return u;
}

__device__ __forceinline__ float norm_x(const GemvNormArgs &p, int i) {
  return norm_x_of(p.mode, p.a[i], p.mode == kGluePlain ? 0.f : p.b[i]);
}

// Sum / max over the 64 lanes of a wave: DPP inside each 16-lane row, then
// the four row results (the same order in every wave).
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dppf<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dppf<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dppf<0x141>(v);  // row_half_mirror
  v += dppf<0x140>(v);  // row_mirror
  return (lanef(v, 0) + lanef(v, 16)) + (lanef(v, 32) + lanef(v, 48));
}
__device__ __forceinline__ float wave_max_f(float v) {
  v = fmaxf(v, dppf<0xB1>(v));
  v = fmaxf(v, dppf<0x4E>(v));
  v = fmaxf(v, dppf<0x141>(v));
  v = fmaxf(v, dppf<0x140>(v));
  return fmaxf(fmaxf(lanef(v, 0), lanef(v, 16)), fmaxf(lanef(v, 32), lanef(v, 48)));
}

__device__ __forceinline__ float norm_y(float x, float inv, float g) {
#pragma clang fp contract(off)
  return x * inv * g;
}

template <bool VEC, int NG, int LPR>
__global__ __launch_bounds__(256) void ternary_gemv_norm_kernel(TernaryGemvGroupArgs a,
                                                                GemvNormArgs p) {
  constexpr int kNormGroupsPerThread = NG;
  constexpr int kNormPieces = 64 * NG;  // 16-byte weight pieces per row (K <= 4096 NG)
  constexpr int kNormPiecesPerLane = kNormPieces / LPR;
  constexpr int kRows = 256 / LPR;
  __shared__ uint4 s_act[256 * NG];
  __shared__ float red[4];
  const int tid = threadIdx.x, slot = tid / LPR, j = tid % LPR, lane = tid & 63, wv_id = tid >> 6;
  const int b = blockIdx.x;
  const uint8_t *w = a.weight[0];
  float *out = a.out[0];
  float ws = a.weight_scale[0];
  int m = a.out_features[0], off = 0;
#pragma unroll
  for (int i = 1; i < kMaxGemvGroup; ++i) {
    if (i < a.n && b >= a.wg_off[i]) {
      w = a.weight[i];
      out = a.out[i];
      ws = a.weight_scale[i];
      m = a.out_features[i];
      off = a.wg_off[i];
    }
  }
  const int K = a.in_features, nb = (K + 3) / 4;
  const int row = (b - off) * kRows + slot;
  const long long b0 = (long long)min(row, m - 1) * a.packed_cols;
  // 1. x for groups tid, tid+256 (16 consecutive elements each) and gamma,
  // loaded before the weights: loads return in order, so these small,
  // cache-resident vectors arrive first and the prologue runs while the
  // weights are still in flight.  VEC: K % 16 == 0 and 16-byte aligned
  // vectors, so a group is four float4 loads of each input.
  float x[kNormGroupsPerThread][16], g[kNormGroupsPerThread][16];
  float4 xa[VEC ? kNormGroupsPerThread : 1][4], xb[VEC ? kNormGroupsPerThread : 1][4],
      xg[VEC ? kNormGroupsPerThread : 1][4];
  if (VEC) {
    // One batch of loads, no branches between them: the second operand is a
    // itself when the mode has none; groups past K read group 0 (discarded).
    const float *pb = p.mode == kGluePlain ? p.a : p.b;
#pragma unroll
    for (int q = 0; q < kNormGroupsPerThread; ++q) {
      const int e0 = 16 * (tid + 256 * q);
      const int base = e0 < K ? e0 : 0;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        xa[q][v4] = *reinterpret_cast<const float4 *>(p.a + base + 4 * v4);
        xb[q][v4] = *reinterpret_cast<const float4 *>(pb + base + 4 * v4);
        xg[q][v4] = *reinterpret_cast<const float4 *>(p.gamma + base + 4 * v4);
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weights
  // 2. this lane's weight pieces (in flight during the prologue)
  uint4 wq[kNormPiecesPerLane];
#pragma unroll
  for (int i = 0; i < kNormPiecesPerLane; ++i) {
    const int c = j + LPR * i;
    if (VEC)
      wq[i] = 16 * c < nb ? ld16_nt(w + b0 + 16 * c) : make_uint4(0, 0, 0, 0);
    else
      wq[i] = 16 * c < nb ? load16_bounded(w, b0 + 16 * c, b0 + nb) : make_uint4(0, 0, 0, 0);
  }
  if (VEC) {
#pragma unroll
    for (int q = 0; q < kNormGroupsPerThread; ++q) {
      const bool in = 16 * (tid + 256 * q) < K;
#pragma unroll
      for (int v4 = 0; v4 < 4; ++v4) {
        const float4 u = xa[q][v4], v = xb[q][v4], gv = xg[q][v4];
        x[q][4 * v4] = in ? norm_x_of(p.mode, u.x, v.x) : 0.f;
        x[q][4 * v4 + 1] = in ? norm_x_of(p.mode, u.y, v.y) : 0.f;
        x[q][4 * v4 + 2] = in ? norm_x_of(p.mode, u.z, v.z) : 0.f;
        x[q][4 * v4 + 3] = in ? norm_x_of(p.mode, u.w, v.w) : 0.f;
        g[q][4 * v4] = in ? gv.x : 0.f;
        g[q][4 * v4 + 1] = in ? gv.y : 0.f;
        g[q][4 * v4 + 2] = in ? gv.z : 0.f;
        g[q][4 * v4 + 3] = in ? gv.w : 0.f;
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < kNormGroupsPerThread; ++q) {
      const int e0 = 16 * (tid + 256 * q);
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int i = e0 + e;
        x[q][e] = i < K ? norm_x(p, i) : 0.f;
        g[q][e] = i < K ? p.gamma[i] : 0.f;
      }
    }
  }
  // 3. sum of squares
  float ss = 0.f;
#pragma unroll
  for (int q = 0; q < kNormGroupsPerThread; ++q)
#pragma unroll
    for (int e = 0; e < 16; ++e) ss = fmaf(x[q][e], x[q][e], ss);
  if (p.h_out && b == 0) {
#pragma unroll
    for (int q = 0; q < kNormGroupsPerThread; ++q) {
      const int e0 = 16 * (tid + 256 * q);
      if (VEC) {
        if (e0 < K)
#pragma unroll
          for (int v4 = 0; v4 < 4; ++v4)
            *reinterpret_cast<float4 *>(p.h_out + e0 + 4 * v4) =
                make_float4(x[q][4 * v4], x[q][4 * v4 + 1], x[q][4 * v4 + 2], x[q][4 * v4 + 3]);
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (e0 + e < K) p.h_out[e0 + e] = x[q][e];
      }
    }
  }
  // block sum (4 waves); the same tree in every workgroup
  ss = wave_sum_f(ss);
  if (lane == 0) red[wv_id] = ss;
  __syncthreads();
  const float sum_sq = (red[0] + red[1]) + (red[2] + red[3]);
  const float inv = 1.0f / sqrtf(sum_sq / (float)K + p.eps);
  float mx = 0.f;
#pragma unroll
  for (int q = 0; q < kNormGroupsPerThread; ++q)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      x[q][e] = norm_y(x[q][e], inv, g[q][e]);  // zero past K (x = 0)
      mx = fmaxf(mx, fabsf(x[q][e]));
    }
  mx = wave_max_f(mx);
  __syncthreads();  // everyone has read red[] as sums
  if (lane == 0) red[wv_id] = mx;
  __syncthreads();
  const float mm = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-5f);
  const float scale = mm / 127.0f, inv_scale = 127.0f / mm;
  // 3. int8 activations into LDS, transposed as the GEMV reads them
#pragma unroll
  for (int q = 0; q < kNormGroupsPerThread; ++q) {
    unsigned d[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      d[t] = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int qv = (int)fminf(fmaxf(roundf(x[q][4 * t + e] * inv_scale), -128.0f), 127.0f);
        d[t] |= (unsigned)(qv & 0xFF) << (8 * e);
      }
    }
    const int gi = tid + 256 * q;
    s_act[(gi & 3) * kNormPieces + (gi >> 2)] = transpose_bytes(make_uint4(d[0], d[1], d[2], d[3]));
  }
  __syncthreads();
  // 4. the projection
  int acc = 0;
#pragma unroll
  for (int i = 0; i < kNormPiecesPerLane; ++i) {
    const int c = j + LPR * i;
    if (16 * c < nb) {
      acc = dot16(wq[i].x, s_act[c], acc);
      acc = dot16(wq[i].y, s_act[kNormPieces + c], acc);
      acc = dot16(wq[i].z, s_act[2 * kNormPieces + c], acc);
      acc = dot16(wq[i].w, s_act[3 * kNormPieces + c], acc);
    }
  }
  acc = lane_group_sum_i<LPR>(acc);
  // combined_scale = weight_scale * act_scale / 127.0 (gemv.rs:297), act_scale = scale * 127
  const float t = ws * (scale * 127.0f);
  const float cs = t / 127.0f;
  if (j == 0 && row < m) out[row] = (float)acc * cs;
}

}  // namespace

hipError_t launch_ternary_gemv_norm(const TernaryGemvGroupArgs &a, const GemvNormArgs &p, bool vec,
                                    hipStream_t s) {
  const int wgs = a.wg_off[a.n];
  if (wgs <= 0) return hipSuccess;
  if (a.in_features > kNormK) return hipErrorInvalidValue;
  const bool one = a.in_features <= kNormK / 2;
  auto go = [&](auto kern) { kern<<<dim3(wgs), dim3(256), 0, s>>>(a, p); };
  switch (p.rows) {
    case 16:
      if (vec) one ? go(ternary_gemv_norm_kernel<true, 1, 16>) : go(ternary_gemv_norm_kernel<true, 2, 16>);
      else one ? go(ternary_gemv_norm_kernel<false, 1, 16>) : go(ternary_gemv_norm_kernel<false, 2, 16>);
      break;
    case 32:
      if (vec) one ? go(ternary_gemv_norm_kernel<true, 1, 8>) : go(ternary_gemv_norm_kernel<true, 2, 8>);
      else one ? go(ternary_gemv_norm_kernel<false, 1, 8>) : go(ternary_gemv_norm_kernel<false, 2, 8>);
      break;
    case 64:
      if (vec) one ? go(ternary_gemv_norm_kernel<true, 1, 4>) : go(ternary_gemv_norm_kernel<true, 2, 4>);
      else one ? go(ternary_gemv_norm_kernel<false, 1, 4>) : go(ternary_gemv_norm_kernel<false, 2, 4>);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ternary_gemv_group(const TernaryGemvGroupArgs &a, bool vec, hipStream_t s) {
  const int wgs = a.wg_off[a.n];
  if (wgs <= 0) return hipSuccess;
  if (vec)
    ternary_gemv_group_kernel<true><<<dim3(wgs), dim3(256), 0, s>>>(a);
  else
    ternary_gemv_group_kernel<false><<<dim3(wgs), dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_ternary_gemv(const TernaryGemvArgs &a, bool vec, hipStream_t s) {
  if (a.out_features <= 0) return hipSuccess;
  const dim3 grid((a.out_features + kRowsPerWg - 1) / kRowsPerWg);
  if (vec)
    ternary_gemv_kernel<true><<<grid, dim3(256), 0, s>>>(a);
  else
    ternary_gemv_kernel<false><<<grid, dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace bnr

// ---------------------------------------------------------------------------
// LM head with i8 weights (CpuBackend::lm_head_matmul_i8_into,
// bitnet-cpu/src/lib.rs:544-575): out[v] = (sum_k w[v][k] * h[k]) * scale[v],
// w int8 [vocab x K], h f32 [K].  One HBM stream of vocab*K bytes (328 MB at
// 128256 x 2560): a workgroup owns 128 rows (8 blocks of 16 rows, 16 lanes
// per row, 16-byte pieces j, j+16, ... per lane) so that the hidden vector,
// staged in LDS once per pass of 4096 values, is reused over 320 KB of
// weights; the next block's pieces are loaded while the current block is
// multiplied.  fp32 products and sums (any order; the reference's AVX2 lane
// order is not reproduced, results agree to rounding).
// ---------------------------------------------------------------------------
namespace bnr {
namespace {

constexpr int kLmBlocks = 8;                     // row blocks of 16 per workgroup
constexpr int kLmPass = 4096;                    // hidden values per LDS pass
constexpr int kLmPieces = kLmPass / 16;          // 16-weight pieces per row and pass
constexpr int kLmPiecesPerLane = kLmPieces / 16;

__device__ __forceinline__ float row_sum16_f(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// acc += the 4 signed bytes of d times h.x .. h.w
__device__ __forceinline__ float fma4_i8(unsigned d, float4 h, float acc) {
  acc = fmaf((float)(int)(signed char)(d & 0xFF), h.x, acc);
  acc = fmaf((float)(int)(signed char)((d >> 8) & 0xFF), h.y, acc);
  acc = fmaf((float)(int)(signed char)((d >> 16) & 0xFF), h.z, acc);
  acc = fmaf((float)((int)d >> 24), h.w, acc);
  return acc;
}

// VEC: rows 16-byte aligned (K % 16 == 0, weights aligned).
template <bool VEC>
__global__ __launch_bounds__(256) void lm_head_i8_kernel(LmHeadArgs a) {
  // hidden values 16c + 4t .. 16c + 4t + 3 of the pass at s_h[t * kLmPieces + c]
  __shared__ float4 s_h[kLmPass / 4];
  const int tid = threadIdx.x, slot = tid >> 4, j = tid & 15;
  const long long row0 = (long long)blockIdx.x * (16 * kLmBlocks) + slot;
  float acc[kLmBlocks][2];
#pragma unroll
  for (int b = 0; b < kLmBlocks; ++b) acc[b][0] = acc[b][1] = 0.f;
  for (int k0 = 0; k0 < a.hidden_size; k0 += kLmPass) {
    const int kn = min(kLmPass, a.hidden_size - k0);
    const int np = (kn + 15) / 16;  // pieces of the pass
    __syncthreads();                // previous pass done with s_h
    for (int g = tid; g < kLmPass / 4; g += 256) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      const int e = 4 * g;
      if (e + 4 <= kn) {
        v = *reinterpret_cast<const float4 *>(a.hidden + k0 + e);
      } else if (e < kn) {
        v.x = a.hidden[k0 + e];
        if (e + 1 < kn) v.y = a.hidden[k0 + e + 1];
        if (e + 2 < kn) v.z = a.hidden[k0 + e + 2];
      }
      s_h[(g & 3) * kLmPieces + (g >> 2)] = v;
    }
    __syncthreads();
    auto load = [&](int b, uint4 *wv) {
      const long long row = min(row0 + 16 * b, (long long)a.vocab_size - 1);
      const int8_t *wr = a.weight + row * a.hidden_size + k0;
#pragma unroll
      for (int i = 0; i < kLmPiecesPerLane; ++i) {
        const int c = j + 16 * i;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (c < np) {
          if (VEC) {
            v = ld16_nt(wr + 16 * c);
          } else {
            unsigned d[4] = {0u, 0u, 0u, 0u};
            for (int q = 0; q < 16; ++q)
              if (16 * c + q < kn) d[q >> 2] |= (unsigned)(uint8_t)wr[16 * c + q] << (8 * (q & 3));
            v = make_uint4(d[0], d[1], d[2], d[3]);
          }
        }
        wv[i] = v;
      }
    };
    uint4 wa[kLmPiecesPerLane], wb[kLmPiecesPerLane];
    load(0, wa);
#pragma unroll
    for (int b = 0; b < kLmBlocks; ++b) {
      uint4 *cur = (b & 1) ? wb : wa;
      uint4 *nxt = (b & 1) ? wa : wb;
      if (b + 1 < kLmBlocks) load(b + 1, nxt);
#pragma unroll
      for (int i = 0; i < kLmPiecesPerLane; ++i) {
        const int c = j + 16 * i;
        if (c < np) {
          acc[b][0] = fma4_i8(cur[i].x, s_h[c], acc[b][0]);
          acc[b][1] = fma4_i8(cur[i].y, s_h[kLmPieces + c], acc[b][1]);
          acc[b][0] = fma4_i8(cur[i].z, s_h[2 * kLmPieces + c], acc[b][0]);
          acc[b][1] = fma4_i8(cur[i].w, s_h[3 * kLmPieces + c], acc[b][1]);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < kLmBlocks; ++b) {
    const float s = row_sum16_f(acc[b][0] + acc[b][1]);
    const long long row = row0 + 16 * b;
    if (j == 0 && row < a.vocab_size) a.out[row] = s * a.scales[row];
  }
}

}  // namespace

hipError_t launch_lm_head_i8(const LmHeadArgs &a, bool vec, hipStream_t s) {
  if (a.vocab_size <= 0) return hipSuccess;
  const long long rows_per_wg = 16 * kLmBlocks;
  const dim3 grid((unsigned)((a.vocab_size + rows_per_wg - 1) / rows_per_wg));
  if (vec)
    lm_head_i8_kernel<true><<<grid, dim3(256), 0, s>>>(a);
  else
    lm_head_i8_kernel<false><<<grid, dim3(256), 0, s>>>(a);
  return hipGetLastError();
}

}  // namespace bnr
