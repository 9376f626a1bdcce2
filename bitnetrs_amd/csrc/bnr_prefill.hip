// bnr_prefill.hip -- gfx950 causal flash prefill of the GQA attention hot
// path on the fp32 matrix cores (grid-mapped and persistent launches).
#include <type_traits>

#include "bnr_device.h"
#include "bnr_internal.h"

#include <hip/hip_runtime.h>
#include <math.h>

#include <algorithm>

namespace bnr {
namespace {

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

// Timeline stamps of a measurement build (BNR_TIMELINE): every wave reads
// the 100 MHz real-time counter into its copy of the record (PfStamp) and
// thread 0 stores wave 0's copy when the workgroup ends.  Scheduling
// barriers keep each read between the instructions of the phases it
// separates.  Product builds compile the stamps away.
#if defined(BNR_TIMELINE)
#define PF_STAMP(st, k)                                                  \
  do {                                                                   \
    __builtin_amdgcn_sched_barrier(0);                                   \
    if (st) (st)[k] = __builtin_amdgcn_s_memrealtime();                  \
    __builtin_amdgcn_sched_barrier(0);                                   \
  } while (0)
#else
#define PF_STAMP(st, k) ((void)0)
#endif

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
  if (a.balanced) {
    pf_bal_map(a, y, it.qt, it.ch, it.nch);
    const int A = (a.start_pos + 31) / 32 + 1;
    it.base = (int)(pf_ceil_sum(it.qt - 1 + A, a.chunk_tiles) - pf_ceil_sum(A - 1, a.chunk_tiles));
    it.q0 = it.qt * 32;
    int len;
    pf_bal_range(min(a.start_pos + it.q0 + 31, last_row) / 32 + 1, it.nch, it.ch, it.kt0, len);
    it.nkt = it.kt0 + len;
    return it;
  }
  prefill_map(a, y, it.qt, it.ch, it.nch, it.base);
  it.q0 = it.qt * 32;
  const int kmax = min(a.start_pos + it.q0 + 31, last_row);
  it.kt0 = it.ch * a.chunk_tiles;
  it.nkt = min(kmax / 32 + 1, it.kt0 + a.chunk_tiles);
  return it;
}

// Copy of key tile kt of kv head h: copy j of wave w fills rows 2J, 2J+1
// (J = w*NI + j); lane l takes row 2J + l/32, LDS chunk l%32.  Rows past the
// last cached one repeat it (their keys are masked for every query).  The
// K half (CK), the V half (CV) or both.
template <int G, bool CK, bool CV>
__device__ __forceinline__ void pf_copy_rows(const PrefillArgs &a, int h, int kt, float *dk,
                                             float *dv) {
  constexpr int NI = kPrefillTile / 4 / (64 * G);  // 1 KB copies per wave per tile
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int last_row = a.start_pos + a.n_tokens - 1;
  const float *kc = a.k_cache + h * a.kv_stride;
  const float *vc = a.v_cache + h * a.kv_stride;
  if (kt * 32 + 31 <= last_row) {
    // A whole cached tile (one uniform test per tile): the tile's address is
    // uniform and the lane's part a 32-bit offset, so the copies take scalar
    // base + vector offset addressing, no 64-bit vector arithmetic.
    const char *kb = (const char *)(kc + (long long)kt * 32 * kHeadDim);
    const char *vb = (const char *)(vc + (long long)kt * 32 * kHeadDim);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int J = wave * NI + j;
      const int r = 2 * J + hl;
      if (CK) dma16((const float *)(kb + (unsigned)(r * kHeadDim + 4 * (col ^ (r & 15))) * 4u), dk + J * 256);
      if (CV) dma16((const float *)(vb + (unsigned)(r * kHeadDim + 4 * col) * 4u), dv + J * 256);
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < NI; ++j) {
    const int J = wave * NI + j;
    const int r = 2 * J + hl;
    const long long grow = (long long)min(kt * 32 + r, last_row) * kHeadDim;
    if (CK) dma16(kc + grow + 4 * (col ^ (r & 15)), dk + J * 256);
    if (CV) dma16(vc + grow + 4 * col, dv + J * 256);
  }
}
// The K half (dv null) or the V half (dk null) of a tile's copies.
template <int G>
__device__ __forceinline__ void pf_copy_half(const PrefillArgs &a, int h, int kt, float *dk,
                                             float *dv) {
  if (dk) pf_copy_rows<G, true, false>(a, h, kt, dk, nullptr);
  else pf_copy_rows<G, false, true>(a, h, kt, nullptr, dv);
}
template <int G>
__device__ __forceinline__ void pf_copy_tile(const PrefillArgs &a, int h, int kt, float *dk,
                                             float *dv) {
  pf_copy_rows<G, true, true>(a, h, kt, dk, dv);
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

// max(v of lane l, v of lane l ^ 32), in every lane: one v_permlane32_swap
// exchanges the two halves of the wave between two copies of v (no LDS
// round trip, unlike a bpermute); whichever half it moves, the pair's
// maximum is the same.
__device__ __forceinline__ float max_half_swap(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
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

// pf_tile_s with each K row chunk read one group of products ahead of its
// use and the next tile's copies (key tile ktn into nk, nv) issued after the
// products; scheduling barriers keep that order.  With a copy in flight the
// compiler waits for LDS reads with lgkmcnt(0) only, so copies among the K
// reads held every group of products to its own reads (tile 7.1 -> 6.8 us
// with the copies after the products, N = 1024 and 2048 on MI355X).
template <int G>
__device__ __forceinline__ floatx16 pf_tile_s_copy(const float *dk, const float (&qf)[64],
                                                   const PrefillArgs &a, int h, int ktn,
                                                   float *nk, float *nv) {
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  floatx16 S = floatx16{};
  const float *krow = dk + col * kHeadDim + 64 * hl;
  const int sw = col & 15;
  float4 kn = ld4(krow + 4 * sw);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float4 kv = kn;
    if (i < 15) kn = ld4(krow + 4 * ((i + 1) ^ sw));
    __builtin_amdgcn_sched_barrier(0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.x, qf[4 * i], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.y, qf[4 * i + 1], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.z, qf[4 * i + 2], S, 0, 0, 0);
    S = __builtin_amdgcn_mfma_f32_32x32x2f32(kv.w, qf[4 * i + 3], S, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  pf_copy_tile<G>(a, h, ktn, nk, nv);
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
  mb = max_half_swap(mb);
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
                                          floatx16 (&O)[4], float m, float l, int *s_last,
                                          unsigned long long *stamp = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, hl = lane >> 5, col = lane & 31;
  const int g = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = it.h, head = h * G + g;
  if (it.nch > 1) {
    // Partial state of this chunk, 16 bytes per lane and instruction: the
    // float4 k (components 4k .. 4k+3 of O, component c = 16*db + r) of lane
    // `lane` of wave g at float ((k * 64 + lane) * 4) of the slot, then m
    // and l of the lane as a pair at float 64 * 64 + 2 * lane.
    const long long slot = (((long long)h * a.n_items + it.base + it.ch) * G + g) * 66 * 64;
    const __amdgpu_buffer_rsrc_t mine = agent_buf(a.ws + slot);
#pragma unroll
    for (int k = 0; k < 16; ++k)
      st4_agent(mine, (k * 64 + lane) * 16,
                make_float4(O[k >> 2][4 * (k & 3)], O[k >> 2][4 * (k & 3) + 1],
                            O[k >> 2][4 * (k & 3) + 2], O[k >> 2][4 * (k & 3) + 3]));
    st2_agent(mine, 64 * 64 * 4 + 8 * lane, m, l);
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
    PF_STAMP(stamp, kPfTicket);
    if (!last) return;
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // Merge the other chunks into this one's registers (same lane layout).
    for (int c = 0; c < it.nch; ++c) {
      if (c == it.ch) continue;
      const __amdgpu_buffer_rsrc_t src = agent_buf(
          a.ws + (((long long)h * a.n_items + it.base + c) * G + g) * 66 * 64);
      float4 ov[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) ov[k] = ld4_agent(src, (k * 64 + lane) * 16);
      const float2 ml = ld2_agent(src, 64 * 64 * 4 + 8 * lane);
      const float mn = fmaxf(m, ml.x);
      const float sa = fast_exp2(m - mn), sb = fast_exp2(ml.x - mn);
      l = l * sa + ml.y * sb;
      m = mn;
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        floatx16 &o = O[k >> 2];
        const int r = 4 * (k & 3);
        o[r] = o[r] * sa + ov[k].x * sb;
        o[r + 1] = o[r + 1] * sa + ov[k].y * sb;
        o[r + 2] = o[r + 2] * sa + ov[k].z * sb;
        o[r + 3] = o[r + 3] * sa + ov[k].w * sb;
      }
    }
    PF_STAMP(stamp, kPfMerged);
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
  PF_STAMP(stamp, kPfStored);
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
#if defined(BNR_TIMELINE)
  unsigned long long stamp_buf[kTimelineStamps] = {};
  unsigned long long *stamp = stamp_buf;
  PF_STAMP(stamp, kPfEntry);
#else
  unsigned long long *stamp = nullptr;
#endif
  const PfItem it = pf_item(a, blockIdx.x, blockIdx.y);
  // Start: the first tile's K and the Q fragment are waited for; its V
  // lands under the first tile's K products.
  constexpr int NI = kPrefillTile / 4 / (64 * G);  // copies per wave per half tile
  pf_copy_half<G>(a, it.h, it.kt0, sK0, nullptr);
  float qf[64];
  pf_load_q<G>(a, it, qf);
  pf_copy_half<G>(a, it.h, it.kt0, nullptr, sV0);
  pf_scale_q(qf, a.scale_log2);
  // All but this wave's NI V copies, then a bare barrier: a fenced one
  // (__syncthreads) would wait for every copy in flight.
  __builtin_amdgcn_s_waitcnt(0x0F70 | NI);
  __builtin_amdgcn_s_barrier();
  PF_STAMP(stamp, kPfReady);
  floatx16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = floatx16{};
  // m starts finite: in a chunk that is not the first, a query may see no key
  // at all (p = 0 for it throughout, and no -inf - -inf in the rescale).
  float m = -1e30f, l = 0.f;
  auto step = [&](int kt, const float *dk, const float *dv, float *nk, float *nv, bool first) {
    // The next tile's copies go out after this tile's K products (the last
    // tile copies itself again into the free buffers, so that the copy needs
    // no branch).
    const floatx16 S = pf_tile_s_copy<G>(dk, qf, a, it.h, min(kt + 1, it.nkt - 1), nk, nv);
    if (first) {
      // the first tile's V: every wave's copies landed (only the next
      // tile's 2 NI copies of this wave may still be in flight)
      __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * NI));
      __builtin_amdgcn_s_barrier();
    }
    pf_tile_pv(a, it, kt, S, dv, O, m, l);
    wait_vmem();  // this wave's copies of the next tile have landed
    __syncthreads();
  };
  step(it.kt0, sK0, sV0, sK1, sV1, true);
  for (int kt = it.kt0 + 1; kt < it.nkt;) {
    step(kt, sK1, sV1, sK0, sV0, false);
    if (++kt >= it.nkt) break;
    step(kt, sK0, sV0, sK1, sV1, false);
    ++kt;
  }
  PF_STAMP(stamp, kPfTiles);
  pf_finish<G>(a, it, O, m, l, &s_last, stamp);
#if defined(BNR_TIMELINE)
  if (a.timeline && threadIdx.x == 0) {
    if (it.nch == 1) stamp_buf[kPfTicket] = stamp_buf[kPfTiles];
    constexpr int kHwId = 4 | (31 << 11), kXccId = 20 | (15 << 11);  // HW_REG_HW_ID, HW_REG_XCC_ID
    stamp_buf[kPfHwId] = ((unsigned long long)(unsigned)__builtin_amdgcn_s_getreg(kXccId) << 32) |
                         (unsigned)__builtin_amdgcn_s_getreg(kHwId);
    stamp_buf[kPfItem] = (unsigned long long)(it.nkt - it.kt0) | ((unsigned long long)it.nch << 16) |
                         ((unsigned long long)it.qt << 32);
    unsigned long long *rec =
        a.timeline + ((long long)blockIdx.y * gridDim.x + blockIdx.x) * kTimelineStamps;
#pragma unroll
    for (int k = 0; k < kTimelineStamps; ++k) rec[k] = stamp_buf[k];
  }
#endif
}

// ---------------------------------------------------------------------------
// 16-query prefill (v_mfma_f32_16x16x4_f32).  The items, key chunks,
// partial-state slots and merge of the grid-mapped launch, each item run by
// two workgroups: half 0 takes queries q0 .. q0+15 of the item's 32-query
// tile, half 1 q0+16 .. q0+31 (grid x = 2 n_kv, x = 2 h + half).  A
// workgroup is G waves (one per q head of kv head h) x 16 queries sharing
// prefill_kernel's double-buffered K/V tiles; a tile product is half as long
// and needs half the Q fragment.
//
// Lane l: query j = l % 16 of the half, lane group u = l / 16.  S^T (32 keys
// x 16 queries) is two 16x16 blocks b; MFMA step t multiplies K (A: lane l
// holds key 16b + j) by Q^T (B: lane l holds query j) at head dim
// 16 (t/4) + 4u + t%4, so a lane reads one 16-byte chunk of its K row per
// four steps and holds its Q dims as 8 float4s.  Register r of S^T block b
// holds key 16b + 4u + r of query j: exactly the B operand P^T of PV step
// 4b + r, whose A operand V^T takes, for O^T block n (0..7), head dim
// 64 (n/4) + 4 j + n%4 of key row 16b + 4u + r -- two float4 reads of the
// row (dims 4j.. and 64+4j..) feed the eight blocks, and the 16 lanes of a
// lane group read 256 contiguous bytes.  O^T register r of block n holds
// dim 64 (n/4) + 16u + 4r + n%4 of query j.  A query's tile maximum and sum
// span the lanes j, j+16, j+32, j+48 (two lane swaps).
// ---------------------------------------------------------------------------
typedef float floatx4 __attribute__((ext_vector_type(4)));

// max(v) and sum(v) over the lanes l, l^16, l^32, l^48: one
// v_permlane16_swap and one v_permlane32_swap; either copy of a swapped
// pair holds the other row's value, so max / sum of the pair is the pair's.
__device__ __forceinline__ float quad_max(float v) {
  unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
  u = __builtin_bit_cast(unsigned, v);
  const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)s[0]), __builtin_bit_cast(float, (unsigned)s[1]));
}
__device__ __forceinline__ float quad_sum(float v) {
  unsigned u = __builtin_bit_cast(unsigned, v);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
  u = __builtin_bit_cast(unsigned, v);
  const auto s = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)s[0]) + __builtin_bit_cast(float, (unsigned)s[1]);
}

// This lane's Q fragment: dims 16m + 4u + e of query q0h + j, unscaled.
template <int G>
__device__ __forceinline__ void pf16_load_q(const PrefillArgs &a, int h, int q0h, float (&qf)[32]) {
  const int lane = threadIdx.x & 63, j = lane & 15, u = lane >> 4;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qrow = min(q0h + j, a.n_tokens - 1);  // rows past the end are not stored
  const float *qp = a.q + ((long long)qrow * a.n_heads + h * G + g) * kHeadDim + 4 * u;
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float4 v = ld4(qp + 16 * m);
    qf[4 * m] = v.x;
    qf[4 * m + 1] = v.y;
    qf[4 * m + 2] = v.z;
    qf[4 * m + 3] = v.w;
  }
}

// S^T of one key tile (blocks 0 and 1), each K chunk read one group ahead
// of its use, then the next tile's copies issued.
template <int G>
__device__ __forceinline__ void pf16_tile_s_copy(const float *dk, const float (&qf)[32],
                                                 const PrefillArgs &a, int h, int ktn, float *nk,
                                                 float *nv, floatx4 &S0, floatx4 &S1) {
  const int lane = threadIdx.x & 63, j = lane & 15, u = lane >> 4;
  // K rows j and 16 + j; chunk c of a row sits at chunk c ^ (row % 16) = c ^ j
  const float *k0 = dk + j * kHeadDim, *k1 = dk + (16 + j) * kHeadDim;
  S0 = floatx4{};
  S1 = floatx4{};
  float4 n0 = ld4(k0 + 4 * (u ^ j)), n1 = ld4(k1 + 4 * (u ^ j));
#pragma unroll
  for (int m = 0; m < 8; ++m) {
    const float4 c0 = n0, c1 = n1;
    if (m < 7) {
      n0 = ld4(k0 + 4 * ((4 * (m + 1) + u) ^ j));
      n1 = ld4(k1 + 4 * ((4 * (m + 1) + u) ^ j));
    }
    __builtin_amdgcn_sched_barrier(0);
    S0 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.x, qf[4 * m], S0, 0, 0, 0);
    S1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.x, qf[4 * m], S1, 0, 0, 0);
    S0 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.y, qf[4 * m + 1], S0, 0, 0, 0);
    S1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.y, qf[4 * m + 1], S1, 0, 0, 0);
    S0 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.z, qf[4 * m + 2], S0, 0, 0, 0);
    S1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.z, qf[4 * m + 2], S1, 0, 0, 0);
    S0 = __builtin_amdgcn_mfma_f32_16x16x4f32(c0.w, qf[4 * m + 3], S0, 0, 0, 0);
    S1 = __builtin_amdgcn_mfma_f32_16x16x4f32(c1.w, qf[4 * m + 3], S1, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  // The next tile's copies after the products: with a copy in flight the
  // compiler waits for LDS reads with lgkmcnt(0) only, so a copy among the
  // K reads would hold every group of products to its own reads (measured:
  // 3.97 us per tile with the copies before the products, 3.76 after).
  pf_copy_tile<G>(a, h, ktn, nk, nv);
}

// Causal mask, online softmax (lazy rescaling as pf_tile_pv) and
// O^T += V^T P^T for key tile kt of the half starting at query q0h.
__device__ __forceinline__ void pf16_tile_pv(const PrefillArgs &a, int q0h, int kt, floatx4 S0,
                                             floatx4 S1, const float *dv, floatx4 (&O)[8],
                                             float &m, float &l) {
  const int lane = threadIdx.x & 63, j = lane & 15, u = lane >> 4;
  const int kbase = kt * 32;
  // The tile's V fragments, all read before the softmax: V row of PV step
  // st is key 16 (st/4) + 4u + st%4.  (Read one step ahead instead, the
  // next step's registers are the current step's, so each read waits for
  // the products before it and each step then waits for its reads.)
  const float *v0 = dv + 4 * u * kHeadDim + 4 * j;
  float4 va[8], vb[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    const float *vr = v0 + (16 * (st >> 2) + (st & 3)) * kHeadDim;
    va[st] = ld4(vr);
    vb[st] = ld4(vr + 64);
  }
  __builtin_amdgcn_sched_barrier(0);
  float s[8] = {S0[0], S0[1], S0[2], S0[3], S1[0], S1[1], S1[2], S1[3]};  // key 16(i/4) + 4u + i%4
  if (kbase + 31 > a.start_pos + q0h) {  // the tile reaches the causal diagonal
    const int pq = a.start_pos + min(q0h + j, a.n_tokens - 1);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (kbase + 16 * (i >> 2) + 4 * u + (i & 3) > pq) s[i] = -INFINITY;
  }
  float mb = s[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) mb = fmaxf(mb, s[i]);
  mb = quad_max(mb);
  if (__ballot(mb > m + 8.0f) != 0) {
    const float mn = fmaxf(m, mb);
    const float alpha = fast_exp2(m - mn);
    l *= alpha;
#pragma unroll
    for (int n = 0; n < 8; ++n) O[n] *= alpha;
    m = mn;
  }
  float p[8], ls = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    p[i] = fast_exp2(s[i] - m);
    ls += p[i];
  }
  l += ls;  // this lane's keys; the query's sum spans its four lanes
#pragma unroll
  for (int st = 0; st < 8; ++st) {
    O[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[st].x, p[st], O[0], 0, 0, 0);
    O[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[st].y, p[st], O[1], 0, 0, 0);
    O[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[st].z, p[st], O[2], 0, 0, 0);
    O[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[st].w, p[st], O[3], 0, 0, 0);
    O[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[st].x, p[st], O[4], 0, 0, 0);
    O[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[st].y, p[st], O[5], 0, 0, 0);
    O[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[st].z, p[st], O[6], 0, 0, 0);
    O[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb[st].w, p[st], O[7], 0, 0, 0);
  }
}

// End of a half item: as pf_finish, with the half's own ticket ((kv head,
// query tile, half)) and the half's region of the item's partial-state
// slot: float4 k of lane l (register k % 4 of O^T blocks 4 (k/4) ..
// 4 (k/4) + 3) at float (k*64 + l)*4, k < 8, then (m, l) of query j at
// 2048 + 2j -- 2080 floats per wave; half h at 2080 h of the slot's 66 * 64.
template <int G>
__device__ __forceinline__ void pf16_finish(const PrefillArgs &a, const PfItem &it, int half,
                                            int q0h, floatx4 (&O)[8], float m, float l,
                                            int *s_last, unsigned long long *stamp = nullptr) {
  const int tid = threadIdx.x, lane = tid & 63, j = lane & 15, u = lane >> 4;
  const int g = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int h = it.h, head = h * G + g;
  l = quad_sum(l);  // the query's sum over its four lanes
  if (it.nch > 1) {
    const long long slot =
        (((long long)h * a.n_items + it.base + it.ch) * G + g) * 66 * 64 + 2080LL * half;
    const __amdgpu_buffer_rsrc_t mine = agent_buf(a.ws + slot);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int n0 = 4 * (k >> 2), r = k & 3;
      st4_agent(mine, (k * 64 + lane) * 16,
                make_float4(O[n0][r], O[n0 + 1][r], O[n0 + 2][r], O[n0 + 3][r]));
    }
    if (u == 0) st2_agent(mine, 2048 * 4 + 8 * j, m, l);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
    __syncthreads();
    unsigned *ctr = a.counters + (((long long)h * a.n_qtiles + it.qt) * 2 + half) * kCounterStride;
    if (tid == 0) {
      const unsigned ticket =
          __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *s_last = ticket == (unsigned)(it.nch - 1);
    }
    __syncthreads();
    const bool last = *s_last;
    __syncthreads();
    PF_STAMP(stamp, kPfTicket);
    if (!last) return;
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int c = 0; c < it.nch; ++c) {
      if (c == it.ch) continue;
      const __amdgpu_buffer_rsrc_t src = agent_buf(
          a.ws + (((long long)h * a.n_items + it.base + c) * G + g) * 66 * 64 + 2080LL * half);
      float4 ov[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) ov[k] = ld4_agent(src, (k * 64 + lane) * 16);
      const float2 ml = ld2_agent(src, 2048 * 4 + 8 * j);
      const float mn = fmaxf(m, ml.x);
      const float sa = fast_exp2(m - mn), sb = fast_exp2(ml.x - mn);
      l = l * sa + ml.y * sb;
      m = mn;
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int n0 = 4 * (k >> 2), r = k & 3;
        O[n0][r] = O[n0][r] * sa + ov[k].x * sb;
        O[n0 + 1][r] = O[n0 + 1][r] * sa + ov[k].y * sb;
        O[n0 + 2][r] = O[n0 + 2][r] * sa + ov[k].z * sb;
        O[n0 + 3][r] = O[n0 + 3][r] * sa + ov[k].w * sb;
      }
    }
    PF_STAMP(stamp, kPfMerged);
  }
  const float inv = 1.0f / l;
  if (q0h + j < a.n_tokens) {
    float *op = a.out + ((long long)(q0h + j) * a.n_heads + head) * kHeadDim + 16 * u;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        st4(op + 64 * hh + 4 * r, make_float4(O[4 * hh][r] * inv, O[4 * hh + 1][r] * inv,
                                              O[4 * hh + 2][r] * inv, O[4 * hh + 3][r] * inv));
  }
  PF_STAMP(stamp, kPfStored);
}

// Piece of a paired launch for this workgroup (PrefillArgs::pair_piece):
// false for a workgroup past the plan's bins or on an empty slot.
__device__ __forceinline__ bool pf16_pair_piece(const PrefillArgs &a, PfItem &it, int &half) {
  const int cu = (int)blockIdx.x % a.pair_cu, slot = (int)blockIdx.x / a.pair_cu;
  // CUs numbered XCD by XCD (workgroup i runs on XCD i % 8) and a kv head's
  // bins on consecutive ones, so that an XCD's L2 holds the K/V of at most
  // two heads (5 heads on 8 XCDs) rather than of every head.
  const int cux = (a.pair_cu & 7) == 0 ? (cu & 7) * (a.pair_cu >> 3) + (cu >> 3) : cu;
  const int hh = cux / a.pair_bins, bin = cux - hh * a.pair_bins;
  if (hh >= a.n_kv) return false;
  const unsigned w0 = a.pair_piece[2 * bin + slot][0], w1 = a.pair_piece[2 * bin + slot][1];
  const int len = (int)(w1 & 255u);
  if (len == 0) return false;
  it.h = hh;
  it.y = 2 * bin + slot;
  it.kt0 = (int)(w0 & 0xFFFFu);
  it.nkt = it.kt0 + len;
  it.qt = (int)((w0 >> 16) & 0x7FFFu);
  it.q0 = it.qt * 32;
  half = (int)(w0 >> 31);
  it.ch = (int)((w1 >> 8) & 255u);
  it.nch = (int)((w1 >> 16) & 255u);
  it.base = (int)(w1 >> 24);
  return true;
}

template <int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2)))
void prefill16_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float sK0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sK1[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV1[kPrefillTile];
  __shared__ int s_last;
#if defined(BNR_TIMELINE)
  unsigned long long stamp_buf[kTimelineStamps] = {};
  unsigned long long *stamp = stamp_buf;
  PF_STAMP(stamp, kPfEntry);
#else
  unsigned long long *stamp = nullptr;
#endif
  int half;
  PfItem it;
  if (a.pair_bins > 0) {
    if (!pf16_pair_piece(a, it, half)) return;
  } else {
    half = blockIdx.x & 1;
    it = pf_item(a, blockIdx.x >> 1, blockIdx.y);
  }
  const int q0h = it.q0 + 16 * half;
  // A half past the last query: every chunk of it exits here, so its ticket
  // is never taken and stays zero.
  if (q0h >= a.n_tokens) return;
  constexpr int NI = kPrefillTile / 4 / (64 * G);
  pf_copy_half<G>(a, it.h, it.kt0, sK0, nullptr);
  float qf[32];
  pf16_load_q<G>(a, it.h, q0h, qf);
  pf_copy_half<G>(a, it.h, it.kt0, nullptr, sV0);
#pragma unroll
  for (int i = 0; i < 32; ++i) qf[i] *= a.scale_log2;
  __builtin_amdgcn_s_waitcnt(0x0F70 | NI);  // all but this wave's V copies
  __builtin_amdgcn_s_barrier();
  PF_STAMP(stamp, kPfReady);
  floatx4 O[8];
#pragma unroll
  for (int n = 0; n < 8; ++n) O[n] = floatx4{};
  float m = -1e30f, l = 0.f;
  // Every scalar load of the kernel arguments has returned: with one still
  // counted, each wait for LDS reads in the tile loop would have to be
  // lgkmcnt(0) (scalar loads return out of order), not just the older reads.
  __builtin_amdgcn_s_waitcnt(0xC07F);
  auto step = [&](int kt, const float *dk, const float *dv, float *nk, float *nv, bool first) {
    floatx4 S0, S1;
    pf16_tile_s_copy<G>(dk, qf, a, it.h, min(kt + 1, it.nkt - 1), nk, nv, S0, S1);
    if (first) {
      __builtin_amdgcn_s_waitcnt(0x0F70 | (2 * NI));
      __builtin_amdgcn_s_barrier();
    }
    pf16_tile_pv(a, q0h, kt, S0, S1, dv, O, m, l);
    // the wait for the next tile's copies stays after the products
    __builtin_amdgcn_sched_barrier(0);
    wait_vmem();
    __syncthreads();
  };
  step(it.kt0, sK0, sV0, sK1, sV1, true);
  for (int kt = it.kt0 + 1; kt < it.nkt;) {
    step(kt, sK1, sV1, sK0, sV0, false);
    if (++kt >= it.nkt) break;
    step(kt, sK0, sV0, sK1, sV1, false);
    ++kt;
  }
  PF_STAMP(stamp, kPfTiles);
  pf16_finish<G>(a, it, half, q0h, O, m, l, &s_last, stamp);
#if defined(BNR_TIMELINE)
  if (a.timeline && threadIdx.x == 0) {
    if (it.nch == 1) stamp_buf[kPfTicket] = stamp_buf[kPfTiles];
    constexpr int kHwId = 4 | (31 << 11), kXccId = 20 | (15 << 11);  // HW_REG_HW_ID, HW_REG_XCC_ID
    stamp_buf[kPfHwId] = ((unsigned long long)(unsigned)__builtin_amdgcn_s_getreg(kXccId) << 32) |
                         (unsigned)__builtin_amdgcn_s_getreg(kHwId);
    stamp_buf[kPfItem] = (unsigned long long)(it.nkt - it.kt0) | ((unsigned long long)it.nch << 16) |
                         ((unsigned long long)it.qt << 32);
    unsigned long long *rec =
        a.timeline + ((long long)blockIdx.y * gridDim.x + blockIdx.x) * kTimelineStamps;
#pragma unroll
    for (int k = 0; k < kTimelineStamps; ++k) rec[k] = stamp_buf[k];
  }
#endif
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
// ---------------------------------------------------------------------------
// Stream-K prefill.  A launch's work is U = n_kv * T units, one unit being a
// (kv head, query tile, key tile) tile product, T the key tiles of all query
// tiles of a head.  Units are ordered (kv head, query tile, key tile) and
// workgroup w of P takes units [w*U/P, (w+1)*U/P): the same number of tile
// products (+-1) for every workgroup, so the resident workgroups of a
// launch finish together, with no tail of short items.  A workgroup's run
// is a sequence of segments: the key tiles of one query tile that fall in
// the run.  A segment holding a whole query tile writes its output; the
// others store their partial state with plain stores -- slot 2w for the
// run's first segment, 2w+1 for its last -- and a second, short launch
// (prefill_sk_merge_kernel) merges the parts of each split query tile: its
// workgroup finds the parts' workgroups wf..wl with sk_wg_of and reads
// their slots.  No tickets or counters are involved.  As in the persistent
// kernel, the next segment's first K/V tile and Q fragment are loaded
// during the current segment's last tile.
//
// Workgroup index -> run: runs go to the XCDs in blocks (XCD x, which gets
// workgroups x, x+8, ..., runs the x-th eighth of the units), so that one
// XCD's L2 sees the K/V tiles of few kv heads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ PfItem sk_item(const SkSeg &sg) {
  PfItem it{};
  it.h = sg.h;
  it.qt = sg.qt;
  it.q0 = 32 * sg.qt;
  it.kt0 = sg.kt0;
  it.nkt = sg.kt1;
  return it;
}

// Output of a whole query tile (normalised O^T, lane layout of pf_finish).
template <int G>
__device__ __forceinline__ void sk_store_out(const PrefillArgs &a, int h, int qt,
                                             const floatx16 (&O)[4], float l) {
  const int lane = threadIdx.x & 63, hl = lane >> 5, col = lane & 31;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q0 = 32 * qt;
  const float inv = 1.0f / (l + __shfl_xor(l, 32));
  if (q0 + col < a.n_tokens) {
    float *op = a.out + ((long long)(q0 + col) * a.n_heads + h * G + g) * kHeadDim + 16 * hl;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      st4(op + 32 * (r >> 2) + 4 * (r & 3),
          make_float4(O[0][r] * inv, O[1][r] * inv, O[2][r] * inv, O[3][r] * inv));
  }
}

// Partial state of a split query tile in slot `slot`: 16 float4 of O per
// lane (register r of the four dim blocks), then (m, l); lane-contiguous.
// Plain stores: the merge runs in the next kernel.
__device__ __forceinline__ float *sk_slot(const PrefillArgs &a, int slot, int G, int g) {
  return a.ws + ((long long)slot * G + g) * 66 * 64;
}

// End of a segment: a whole query tile writes its output; a part of a split
// one stores its partial state for prefill_sk_merge_kernel.
template <int G>
__device__ __forceinline__ void sk_finish(const PrefillArgs &a, const SkSeg &sg, int w,
                                          const floatx16 (&O)[4], float m, float l) {
  if (sg.kt0 == 0 && sg.kt1 == sg.nk) {
    sk_store_out<G>(a, sg.h, sg.qt, O, l);
    return;
  }
  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = 2 * w + (sk_u0(w, a.sk_units, gridDim.x) >= sg.qstart ? 0 : 1);
  float *p = sk_slot(a, slot, G, g);
#pragma unroll
  for (int r = 0; r < 16; ++r)
    st4(p + (r * 64 + lane) * 4, make_float4(O[0][r], O[1][r], O[2][r], O[3][r]));
  *reinterpret_cast<float2 *>(p + 64 * 64 + lane * 2) = make_float2(m, l);
}

// Merge of the split query tiles of a stream-K launch (P = its workgroup
// count): workgroup (qt, h), wave g merges the parts wf..wl of query tile qt
// of kv head h, head g, in run order, and writes the output.  Query tiles
// that one run held whole were written by it; their workgroups exit.
template <int G>
__global__ __launch_bounds__(64 * G) void prefill_sk_merge_kernel(PrefillArgs a, int P) {
  const int qt = blockIdx.x, h = blockIdx.y;
  const int nqt = a.n_qtiles, A = (a.start_pos + 31) / 32 + 1;
  const int nt_last = (a.start_pos + a.n_tokens - 1) / 32 + 1;
  const int nk = qt + 1 < nqt ? A + qt : nt_last;
  const long long U = a.sk_units;
  const long long qs = (long long)h * a.sk_per_head + sk_off(qt, A);
  const int wf = sk_wg_of(qs, U, P), wl = sk_wg_of(qs + nk - 1, U, P);
  if (wf == wl) return;
  const int lane = threadIdx.x & 63;
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  floatx16 O[4];
  float m = -1e30f, l = 0.f;
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = floatx16{};
  for (int w = wf; w <= wl; ++w) {
    const int slot = 2 * w + (sk_u0(w, U, P) >= qs ? 0 : 1);
    const float *p = sk_slot(a, slot, G, g);
    float4 ov[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) ov[r] = ld4(p + (r * 64 + lane) * 4);
    const float2 ml = *reinterpret_cast<const float2 *>(p + 64 * 64 + lane * 2);
    const float mn = fmaxf(m, ml.x);
    const float sa = fast_exp2(m - mn), sb = fast_exp2(ml.x - mn);
    l = l * sa + ml.y * sb;
    m = mn;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      O[0][r] = O[0][r] * sa + ov[r].x * sb;
      O[1][r] = O[1][r] * sa + ov[r].y * sb;
      O[2][r] = O[2][r] * sa + ov[r].z * sb;
      O[3][r] = O[3][r] * sa + ov[r].w * sb;
    }
  }
  sk_store_out<G>(a, h, qt, O, l);
}

template <int G>
__global__ __launch_bounds__(64 * G) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_streamk_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) float sK0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sK1[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV0[kPrefillTile];
  __shared__ __attribute__((aligned(16))) float sV1[kPrefillTile];
  const int P = gridDim.x, b = blockIdx.x;
  const int w = P % 8 == 0 ? (b % 8) * (P / 8) + b / 8 : b;  // XCD b % 8 runs the (b % 8)-th eighth
  const long long U = a.sk_units, u_end = sk_u0(w + 1, U, P);
  long long u = sk_u0(w, U, P);  // first unit of the current segment
  if (u >= u_end) return;
  SkSeg sg = sk_seg(a, u, u_end);
  pf_copy_tile<G>(a, sg.h, sg.kt0, sK0, sV0);
  float qf[64];
  pf_load_q<G>(a, sk_item(sg), qf);
  pf_scale_q(qf, a.scale_log2);
  wait_vmem();
  __syncthreads();
  floatx16 O[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) O[db] = floatx16{};
  float m = -1e30f, l = 0.f;
  int kt = sg.kt0;
  // One tile of the current segment on (dk, dv); the next tile, or the next
  // segment's first, is copied into (nk, nv).  False once the run is done.
  auto step = [&](const float *dk, const float *dv, float *nk, float *nv) -> bool {
    const bool lastt = kt + 1 == sg.kt1;
    const long long un = u + (sg.kt1 - sg.kt0);  // first unit of the next segment
    const bool more = lastt && un < u_end;
    const SkSeg ns = more ? sk_seg(a, un, u_end) : sg;
    if (!lastt) pf_copy_tile<G>(a, sg.h, kt + 1, nk, nv);
    else if (more) pf_copy_tile<G>(a, ns.h, ns.kt0, nk, nv);
    const floatx16 S = pf_tile_s(dk, qf);
    pf_tile_pv(a, sk_item(sg), kt, S, dv, O, m, l);
    if (more) pf_load_q<G>(a, sk_item(ns), qf);  // qf is no longer read by this segment
    if (lastt) sk_finish<G>(a, sg, w, O, m, l);
    wait_vmem();  // this wave's copies (next tile, next Q) have landed
    __syncthreads();
    if (!lastt) {
      ++kt;
      return true;
    }
    if (!more) return false;
    sg = ns;
    u = un;
    kt = sg.kt0;
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
}
#pragma clang diagnostic pop

}  // namespace

void prefill_streamk_units(PrefillArgs &a) {
  const long long nqt = a.n_qtiles, A = (a.start_pos + 31) / 32 + 1;
  const long long nt_last = (a.start_pos + a.n_tokens - 1) / 32 + 1;
  a.sk_per_head = A * (nqt - 1) + (nqt - 1) * (nqt - 2) / 2 + nt_last;
  a.sk_units = a.sk_per_head * a.n_kv;
}

hipError_t launch_prefill_streamk(const PrefillArgs &a, int group, int wgs, hipStream_t s) {
  if (a.n_tokens <= 0) return hipSuccess;
  if (wgs <= 0 || a.sk_units < wgs || !a.ws) return hipErrorInvalidValue;
  const dim3 grid(wgs), mgrid(a.n_qtiles, a.n_kv);
  switch (group) {
    case 2:
      prefill_streamk_kernel<2><<<grid, dim3(128), 0, s>>>(a);
      prefill_sk_merge_kernel<2><<<mgrid, dim3(128), 0, s>>>(a, wgs);
      break;
    case 4:
      prefill_streamk_kernel<4><<<grid, dim3(256), 0, s>>>(a);
      prefill_sk_merge_kernel<4><<<mgrid, dim3(256), 0, s>>>(a, wgs);
      break;
    case 8:
      prefill_streamk_kernel<8><<<grid, dim3(512), 0, s>>>(a);
      prefill_sk_merge_kernel<8><<<mgrid, dim3(512), 0, s>>>(a, wgs);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
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
  for (int l = 0; l <= kMaxLptChunk; ++l) a.bal_off[l] = 0;
  if (!a.lpt) {
    a.balanced = 0;
    return;
  }
  if (a.balanced) {
    // chunks per length: a tile of nk key tiles in m chunks has nk % m of
    // length nk / m + 1 (at most ct) and the others of nk / m
    long long cnt[kMaxLptChunk + 2] = {};
    auto add = [&](int nk) {
      const int m = (nk + ct - 1) / ct, q = nk / m, r = nk - q * m;
      cnt[q + 1] += r;
      cnt[q] += m - r;
    };
    add(nt_last);
    for (int qt = 0; qt + 1 < nqt; ++qt) add(qt + A);
    for (int l = ct; l >= 1; --l) a.bal_off[l - 1] = a.bal_off[l] + (int)cnt[l];
  }
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
  if (a.q16) {
    const dim3 grid16 = a.pair_bins > 0 ? dim3(2 * a.pair_cu) : dim3(2 * a.n_kv, a.n_items);
    switch (group) {
      case 2: prefill16_kernel<2><<<grid16, dim3(128), 0, s>>>(a); break;
      case 4: prefill16_kernel<4><<<grid16, dim3(256), 0, s>>>(a); break;
      case 8: prefill16_kernel<8><<<grid16, dim3(512), 0, s>>>(a); break;
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

}  // namespace bnr
