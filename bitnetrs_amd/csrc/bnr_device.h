// bnr_device.h -- device helpers shared by the gfx950 kernels of the
// attention path (wave64): RoPE rotation, DPP row reductions, 16-byte
// loads/stores, agent-coherent accesses.  Included by the .hip sources only.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>

#include "bnr_internal.h"

namespace bnr {

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

// 16 bytes with the non-temporal hint (global_load_dwordx4 ... nt), for
// data read once: the K/V rows of a decode step.  Measured on MI355X: a
// single-sequence step at 4096 rows 9.42 -> 8.60 us, and plain streaming
// reads of the same 21 MB 5.42 -> 4.98 us.
__device__ __forceinline__ float4 ld4_nt(const float *p) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void st4(float *p, float4 v) {
  *reinterpret_cast<float4 *>(p) = v;
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

// The 16- and 8-byte forms of st_agent / ld_agent: buffer stores and loads
// with the sc1 cache policy (device scope), over a raw buffer that starts at
// `base`; offsets in bytes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t agent_buf(const float *base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7fffffff,
                                           0x00020000);
}
__device__ __forceinline__ void st4_agent(__amdgpu_buffer_rsrc_t r, int off, float4 v) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v x = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned, x),
                                         r, off, 0, 16);
}
__device__ __forceinline__ void st2_agent(__amdgpu_buffer_rsrc_t r, int off, float a, float b) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v x = {a, b};
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, x),
                                        r, off, 0, 16);
}
__device__ __forceinline__ float4 ld4_agent(__amdgpu_buffer_rsrc_t r, int off) {
  typedef float f4v __attribute__((ext_vector_type(4)));
  const f4v v = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float2 ld2_agent(__amdgpu_buffer_rsrc_t r, int off) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  const f2v v = __builtin_bit_cast(f2v, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16));
  return make_float2(v.x, v.y);
}

// Host-slice calls: every thread's stores complete, then thread 0 stores seq
// into a pinned host word with a system-scope release, so the workgroup's
// outputs reach the host before the word does.  All threads must call it.
__device__ __forceinline__ void signal_host(unsigned *word, unsigned seq) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_store(word, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Device-scope float add whose result is not used: one global_atomic_add_f32
// (device memory is coarse-grained; the library is built with
// -munsafe-fp-atomics so that this is not a compare-and-swap loop).
__device__ __forceinline__ void add_agent(float *p, float v) {
  (void)__hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace bnr
