// bnr_glue.hip -- gfx950 kernels of the layer glue around the projections:
// RMSNorm (bitnet-cpu/src/norm.rs:76-136), per-token absmax int8
// quantisation (bitnet-core/src/quant/absmax.rs:127-170), the squared-ReLU
// gate (bitnet-cpu/src/lib.rs:494-509) and the residual add
// (bitnet-model/src/lib.rs:1061,1130), fused so that a decode layer needs one
// launch between two projections.
//
// norm_quant_kernel: one workgroup of 1024 lanes per vector.  Each lane keeps
// up to 8 elements in registers (n <= 8192, every projection input of the 2B
// model); longer vectors are re-read from memory in each phase.
//   x     = a | a + b (written to h_out) | max(a,0)^2 * b      (mode)
//   y     = (x * (1/sqrt(sum(x^2)/n + eps))) * gamma             (optional norm)
//   q     = clamp(round(y * 127/m), -128, 127), m = max(max|y|, 1e-5)
// The sum of squares is a tree (not the reference's 8-lane AVX2 order), so y
// agrees with the reference to rounding; given y, q and the scales are
// computed exactly as the reference does (one f32 multiply, round half away
// from zero, correctly rounded division and square root).
#include "bnr_device.h"
#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

namespace bnr {
namespace {

constexpr int kNormLanes = 1024;
constexpr int kNormCache = 8;

__device__ __forceinline__ float wave_sum_f(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// Block-wide sum / max over the 16 waves (every lane gets the result).
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum_f(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kNormLanes / 64; ++i) s += red[i];
  return s;
}
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max_f(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < kNormLanes / 64; ++i) m = fmaxf(m, red[i]);
  return m;
}

__device__ __forceinline__ float glue_x(const NormQuantArgs &a, int i) {
#pragma clang fp contract(off)
  const float u = a.a[i];
  if (a.mode == kGlueResidual) return u + a.b[i];
  if (a.mode == kGlueSqrelu) {
    const float r = fmaxf(u, 0.0f);  // max(NaN, 0) = 0, as _mm256_max_ps(g, 0)
    return r * r * a.b[i];
  }
  return u;
}

__device__ __forceinline__ float glue_y(float x, float inv, float g) {
#pragma clang fp contract(off)
  return x * inv * g;
}

__global__ __launch_bounds__(kNormLanes) void norm_quant_kernel(NormQuantArgs a) {
  __shared__ float red[kNormLanes / 64];
  const int tid = threadIdx.x;
  const bool cached = a.n <= kNormLanes * kNormCache;
  float v[kNormCache], gm[kNormCache];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const int i = tid + kNormLanes * k;
    gm[k] = a.gamma && i < a.n ? a.gamma[i] : 1.0f;
  }
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const int i = tid + kNormLanes * k;
    v[k] = 0.f;
    if (i < a.n) {
      v[k] = glue_x(a, i);
      if (a.h_out) a.h_out[i] = v[k];
      ss = fmaf(v[k], v[k], ss);
    }
  }
  if (!cached)
    for (int i = tid + kNormLanes * kNormCache; i < a.n; i += kNormLanes) {
      const float x = glue_x(a, i);
      if (a.h_out) a.h_out[i] = x;
      ss = fmaf(x, x, ss);
    }
  float inv = 1.0f;
  if (a.gamma) {
    const float sum_sq = block_sum(ss, red);
    const float rms = sqrtf(sum_sq / (float)a.n + a.eps);
    inv = 1.0f / rms;
  }
  // phase 2: y, max |y|
  float mx = 0.f;
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const int i = tid + kNormLanes * k;
    if (i < a.n) {
      if (a.gamma) v[k] = glue_y(v[k], inv, gm[k]);
      if (a.y_out) a.y_out[i] = v[k];
      mx = fmaxf(mx, fabsf(v[k]));
    }
  }
  if (!cached)
    for (int i = tid + kNormLanes * kNormCache; i < a.n; i += kNormLanes) {
      float y = a.h_out ? a.h_out[i] : glue_x(a, i);
      if (a.gamma) y = glue_y(y, inv, a.gamma[i]);
      if (a.y_out) a.y_out[i] = y;
      mx = fmaxf(mx, fabsf(y));
    }
  if (!a.q_out) {
    if (a.done) signal_host(a.done, a.seq);
    return;
  }
  const float m = fmaxf(block_max(mx, red), 1e-5f);  // f32::max(max_abs, ABSMAX_MIN)
  const float scale = m / 127.0f;
  const float inv_scale = 127.0f / m;
  if (tid == 0) {
    if (a.scale_out) *a.scale_out = scale;
    if (a.act_absmax) *a.act_absmax = scale * 127.0f;  // q_scale * 127.0 (bitnet-model/src/lib.rs:642)
  }
#pragma unroll
  for (int k = 0; k < kNormCache; ++k) {
    const int i = tid + kNormLanes * k;
    if (i < a.n) a.q_out[i] = (int8_t)fminf(fmaxf(roundf(v[k] * inv_scale), -128.0f), 127.0f);
  }
  if (!cached)
    for (int i = tid + kNormLanes * kNormCache; i < a.n; i += kNormLanes) {
      float y = a.h_out ? a.h_out[i] : glue_x(a, i);
      if (a.gamma) y = glue_y(y, inv, a.gamma[i]);
      a.q_out[i] = (int8_t)fminf(fmaxf(roundf(y * inv_scale), -128.0f), 127.0f);
    }
  if (a.done) signal_host(a.done, a.seq);
}

// out = (max(gate,0)^2) * up, elementwise (CpuBackend::sqrelu_gate).
__global__ __launch_bounds__(256) void sqrelu_kernel(const float *gate, const float *up, float *out,
                                                     long long n, unsigned *done, unsigned seq) {
#pragma clang fp contract(off)
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256) {
    const float r = fmaxf(gate[i], 0.0f);
    out[i] = r * r * up[i];
  }
  if (done) signal_host(done + blockIdx.x, seq);
}

// h += delta (axpy_f32_fast(1.0, delta, h): one rounding per element).
__global__ __launch_bounds__(256) void residual_kernel(float *h, const float *delta, long long n) {
  for (long long i = blockIdx.x * 256LL + threadIdx.x; i < n; i += (long long)gridDim.x * 256)
    h[i] = h[i] + delta[i];
}

}  // namespace

hipError_t launch_norm_quant(const NormQuantArgs &a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  norm_quant_kernel<<<dim3(1), dim3(kNormLanes), 0, s>>>(a);
  return hipGetLastError();
}

hipError_t launch_sqrelu(const float *gate, const float *up, float *out, long long n, hipStream_t s,
                         unsigned *done, unsigned seq) {
  if (n <= 0) return hipSuccess;
  const long long blocks = sqrelu_blocks(n);
  sqrelu_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(gate, up, out, n, done, seq);
  return hipGetLastError();
}

hipError_t launch_residual(float *h, const float *delta, long long n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const long long blocks = std::min<long long>((n + 255) / 256, 4096);
  residual_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(h, delta, n);
  return hipGetLastError();
}

}  // namespace bnr
