// bnr_api.cpp -- C ABI of the gfx950 GQA attention path (include/bitnet_hip.h).
//
// This is the host side of the backend: argument validation in the
// reference's order and with its error kinds, the lazily built RoPE table,
// the HBM mirrors of host KV caches behind the trait-shaped entry points,
// the split-K decode planner and the workspace.  Kernels live in
// bnr_kernels.hip.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <list>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/bitnet_hip.h"
#include "bnr_internal.h"

using namespace bnr;

// ---------------------------------------------------------------------------
// Errors: the calling thread's last error, kept both as BitNetError's Display
// text and as the fields of its variant (bitnet-core/src/error.rs:12-55), so
// that a binding can rebuild the variant itself:
//   InvalidShape { expected, got }       first = expected, second = got
//   InvalidConfig(String)                first = the message
//   BackendError { backend, message }    first = "HIP", second = the message
//   UnsupportedDevice(String)            first = the message
//   QuantizationError(String)            first = the message
// ---------------------------------------------------------------------------
namespace {
struct LastError {
  int kind = BNR_OK;
  std::string text, first, second;
};
}  // namespace
static thread_local LastError g_err;

static int set_err(int kind, std::string text, std::string first, std::string second) {
  g_err.kind = kind;
  g_err.text = std::move(text);
  g_err.first = std::move(first);
  g_err.second = std::move(second);
  return kind;
}

static int set_ok() {
  g_err = LastError();
  return BNR_OK;
}

static int err_shape(const std::string &expected, const std::string &got) {
  return set_err(BNR_INVALID_SHAPE, "invalid tensor shape: expected " + expected + ", got " + got,
                 expected, got);
}

static std::string fmt(const char *f, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(buf, sizeof buf, f, ap);
  va_end(ap);
  return buf;
}

static int err_config(const std::string &msg) {
  return set_err(BNR_INVALID_CONFIG, "invalid model configuration: " + msg, msg, "");
}

static int err_backend(const std::string &msg) {
  return set_err(BNR_BACKEND_ERROR, "backend error (HIP): " + msg, "HIP", msg);
}

static int err_quant(const std::string &msg) {
  return set_err(BNR_QUANTIZATION_ERROR, "quantization error: " + msg, msg, "");
}

static int err_device(const std::string &msg) {
  return set_err(BNR_UNSUPPORTED_DEVICE, "unsupported device: " + msg, msg, "");
}

// Rust's Display of an f32: the shortest decimal that reads back to the same
// value, written positionally ("0.5", "-3", "0.0000001", "NaN", "inf").
static std::string rust_f32(float x) {
  if (std::isnan(x)) return "NaN";
  if (std::isinf(x)) return x < 0 ? "-inf" : "inf";
  if (x == 0.0f) return std::signbit(x) ? "-0" : "0";
  char e[64];
  int p = 1;
  for (; p <= 9; ++p) {
    snprintf(e, sizeof e, "%.*e", p - 1, (double)x);
    if ((float)strtod(e, nullptr) == x) break;
  }
  std::string digits;
  const bool neg = e[0] == '-';
  const char *q = e + (neg ? 1 : 0);
  for (; *q && *q != 'e'; ++q)
    if (*q != '.') digits += *q;
  const int ex = atoi(q + 1);
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  const int nd = (int)digits.size();
  std::string out = neg ? "-" : "";
  if (ex >= nd - 1) {
    out += digits + std::string((size_t)(ex - (nd - 1)), '0');
  } else if (ex >= 0) {
    out += digits.substr(0, (size_t)ex + 1) + "." + digits.substr((size_t)ex + 1);
  } else {
    out += "0." + std::string((size_t)(-ex - 1), '0') + digits;
  }
  return out;
}

static int err_hip(hipError_t e, const char *what) {
  return err_backend(std::string(what) + ": " + hipGetErrorString(e));
}

#define HIP_TRY(expr, what)                 \
  do {                                      \
    hipError_t e_ = (expr);                 \
    if (e_ != hipSuccess) return err_hip(e_, what); \
  } while (0)

// ---------------------------------------------------------------------------
// Context
// ---------------------------------------------------------------------------
namespace {

// HBM copy of one host KV cache (one layer), for bnr_masked_attention.
struct Mirror {
  const float *hk = nullptr, *hv = nullptr;
  size_t k_len = 0, v_len = 0, n_kv = 0, head_dim = 0;
  size_t rows = 0;    // rows per kv head held on the device
  size_t synced = 0;  // rows 0..synced-1 match the host
  float *dk = nullptr, *dv = nullptr;
  std::vector<float> probe;  // kv_probe of the host rows at the last sync
};

// Samples of rows 0, (n-1)/2 and n-1 of every kv head of a host cache: the
// first and last four floats of the k and v rows.  Taken when a mirror is
// synced to n rows; the next call uploads only its new row if they still
// match, and re-uploads every row if one of them was rewritten since.  A
// rewrite of any other row goes unseen and needs bnr_mirror_invalidate.
void kv_probe(const float *k, const float *v, size_t n_kv, size_t head_stride, size_t head_dim,
              size_t n, std::vector<float> &out) {
  out.clear();
  if (n == 0) return;
  const size_t c = std::min<size_t>(4, head_dim);
  const size_t rows[3] = {0, (n - 1) / 2, n - 1};
  for (size_t kh = 0; kh < n_kv; ++kh)
    for (size_t r : rows)
      for (const float *src : {k, v}) {
        const float *row = src + kh * head_stride + r * head_dim;
        out.insert(out.end(), row, row + c);
        out.insert(out.end(), row + head_dim - c, row + head_dim);
      }
}

// HBM copy of one host ternary weight matrix, for bnr_ternary_gemv_preq.
// The fingerprint (64 bytes sampled across the buffer) catches a different
// matrix placed at the same address with the same length, which a freed and
// reallocated host buffer can be; rewriting weights in place still needs
// bnr_mirror_invalidate.
constexpr int kFingerprint = 64;
struct WeightMirror {
  const uint8_t *host = nullptr;
  size_t len = 0;
  uint8_t *dev = nullptr;
  uint8_t print[kFingerprint] = {};
};

void fingerprint(const uint8_t *p, size_t len, uint8_t *out) {
  for (int i = 0; i < kFingerprint; ++i)
    out[i] = p[len > 1 ? (size_t)i * (len - 1) / (kFingerprint - 1) : 0];
}

constexpr size_t kMaxWeightMirrors = 1024;

struct PrefillPlanEntry {
  int n_tokens, start_pos, n_kv, pair_pref;
  long long cap;
  PrefillChoice choice;
  PairPlan pairs;  // choice.pairs
};

struct DeviceGuard {
  int prev = -1;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) (void)hipSetDevice(dev);
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

constexpr size_t kMaxMirrors = 256;

// Tiled prefill launches: planned key chunks on a grid of items, the same
// items from a queue of resident workgroups, stream-K runs, or (auto, the
// default) stream-K or the grid by shape.
constexpr int kPrefillGrid = 0, kPrefillQueue = 1, kPrefillStreamK = 2, kPrefillAuto = 3;

// Merge state of split-K decode launches: split partials (exact path),
// tickets and reference-merge accumulators.  Kernels leave tickets and
// accumulators at zero after every launch; launches that share a workspace
// must be ordered (one stream, or synchronised).
struct DecodeWs {
  float *ws_o = nullptr;
  size_t ws_o_floats = 0;
  float2 *ws_ml = nullptr;
  size_t ws_ml_n = 0;
  unsigned *counters = nullptr;
  size_t n_counters = 0;
  float *acc = nullptr;  // reference-merge accumulators
  size_t acc_floats = 0;
  float *scores = nullptr;  // generic kernel: scores of every row
  size_t scores_floats = 0;
  float *rot = nullptr;  // other shapes: rotated copies of q and k
  size_t rot_floats = 0;
};

}  // namespace

struct bnr_ctx {
  int device = 0;
  std::string name;
  std::mutex mu;
  hipStream_t stream = nullptr;  // stream of the synchronous host entry points

  // RoPE table (CpuBackend::rope_cache policy, bitnet-cpu/src/lib.rs:79,299-311)
  bool tab_valid = false;
  size_t tab_len = 0, tab_head_dim = 0;
  float tab_theta = 0.f;
  float *d_cos = nullptr, *d_sin = nullptr;

  // Split-K decode workspaces: one for launches on the library's own stream
  // (the host-slice entry points), one for launches on callers' streams (the
  // device entry points), so that the two kinds never share merge state.
  DecodeWs hws, dws;
  float *pf_ws = nullptr;  // prefill chunk partials
  size_t pf_ws_floats = 0;
  unsigned *pf_counters = nullptr;
  size_t n_pf_counters = 0;
  unsigned *pf_queue = nullptr;  // persistent prefill: next item, workgroups done
  size_t n_pf_queue = 0;

  // host-path staging
  float *d_q = nullptr, *d_out = nullptr;
  size_t d_q_n = 0, d_out_n = 0;
  float *h_stage = nullptr;  // pinned host staging of the host-slice calls
  size_t h_stage_n = 0;
  float *h_zc = nullptr;  // zero-copy staging: pinned host memory kernels read and write
  float *d_zc = nullptr;  // its device address
  size_t h_zc_n = 0;
  // Completion words of the host-slice calls: pinned, coherent host memory
  // the kernels store a call's sequence number into (kSignalWords of them).
  unsigned *h_sig = nullptr, *d_sig = nullptr;
  unsigned sig_seq = 0;

  // mirrors, most recently used first
  std::list<Mirror> mirrors;
  std::vector<float> probe_now;  // kv_probe scratch (capacity kept across calls)
  std::list<WeightMirror> weight_mirrors;
  uint8_t *d_bytes = nullptr;  // int8 activation staging
  size_t d_bytes_n = 0;
  int mirror_mode = BNR_MIRROR_INCREMENTAL;

  // decode planner
  int target_wgs = 256;  // small decode launches: at most this many workgroups (the CU count)
  int large_wgs = 1024;
  int force_rpg = 0;
  int min_passes = 1;
  int merge_mode = -1;  // -1: planner decides; 0: second kernel; 1: in-kernel ticket; 2: reference merge;
                        // 3: reference merge, deterministic
  int split_cost = -1;  // planner cost of a split of the in-kernel merges (ns); -1: mode default
  int ref_rows = 0;     // reference merge: rows per split (0: planner)
  int ref_waves = 0;    // reference merge, small launches: 4 or 8 waves, 0: by length

  // measurement builds (BNR_TIMELINE): where decode and grid-mapped prefill
  // launches store their phase stamps (bnr_debug_decode_timeline), or null
  unsigned long long *timeline = nullptr;

  // device scratch of bnr_dev_decode_attention_noalloc (this GPU's copy)
  void *noalloc = nullptr;
  std::string noalloc_err;

  // prefill planner
  int n_cu = 256;
  int pf_chunk_tiles = -1;  // -1: planner decides; else key tiles per chunk
  int pf_mode = kPrefillAuto;  // tiled prefill launch: kPrefillAuto / Grid / Queue / StreamK
  int pf_sk_wgs = 0;              // stream-K workgroups (0: every resident slot)
  int pf_q16 = -1;                // 16-query halves (prefill16_kernel): -1 planner, 0 never, 1 always
  int pf_balanced = -1;           // balanced key chunks: -1 planner, 0 never, 1 always
  // norm-fused GEMV: the most rows per workgroup (16, 32, 64) that keep the
  // launch at or above this many workgroups
  int gemv_norm_min_wgs = 256;
  int pf_pair = -1;               // paired 16-query launches: -1 planner (4 q heads per kv head), 0 never, 1 where possible
  std::vector<PrefillPlanEntry> pf_plans;  // recent (shape -> key tiles per chunk) plans
};

namespace {

void free_mirror(Mirror &m) {
  if (m.dk) (void)hipFree(m.dk);
  if (m.dv) (void)hipFree(m.dv);
  m.dk = m.dv = nullptr;
}

// Grow-only device buffer.
int ensure_buf(float **p, size_t *cap, size_t n, const char *what) {
  if (*cap >= n && *p) return BNR_OK;
  if (*p) {
    (void)hipDeviceSynchronize();
    (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
  }
  size_t want = std::max<size_t>(n, 1024);
  HIP_TRY(hipMalloc((void **)p, want * sizeof(float)), what);
  *cap = want;
  return BNR_OK;
}

size_t round4(size_t n) { return (n + 3) & ~(size_t)3; }

// Grow-only pinned host buffer.  The host-slice entry points gather their
// slices into it and move them with one DMA copy each way; a pageable copy
// pays a staging round trip of its own for every slice.
int ensure_host(bnr_ctx *c, size_t n) {
  if (c->h_stage_n >= n && c->h_stage) return BNR_OK;
  if (c->h_stage) {
    (void)hipStreamSynchronize(c->stream);
    (void)hipHostFree(c->h_stage);
    c->h_stage = nullptr;
    c->h_stage_n = 0;
  }
  const size_t want = std::max<size_t>(n, 16384);
  HIP_TRY(hipHostMalloc((void **)&c->h_stage, want * sizeof(float), hipHostMallocDefault),
          "pinned staging alloc");
  c->h_stage_n = want;
  return BNR_OK;
}

// Host slices to device memory through the pinned buffer: the parts are
// packed back to back and sent with one DMA copy.  The packing is not
// ordered with the stream, so a call uploads once before get_host.
struct HostPart {
  const void *src;
  size_t bytes;
};
int put_host(bnr_ctx *c, void *dev, std::initializer_list<HostPart> parts, const char *what) {
  size_t total = 0;
  for (const HostPart &p : parts) total += p.bytes;
  int st = ensure_host(c, (total + 3) / 4);
  if (st) return st;
  char *h = reinterpret_cast<char *>(c->h_stage);
  for (const HostPart &p : parts) {
    if (p.bytes) std::memcpy(h, p.src, p.bytes);
    h += p.bytes;
  }
  HIP_TRY(hipMemcpyAsync(dev, c->h_stage, total, hipMemcpyHostToDevice, c->stream), what);
  return BNR_OK;
}

// A device range into a host slice through the pinned buffer.  Waits for
// the stream: the host entry points return with their outputs written.
int get_host(bnr_ctx *c, void *host, const void *dev, size_t bytes, const char *what) {
  int st = ensure_host(c, (bytes + 3) / 4);
  if (st) return st;
  HIP_TRY(hipMemcpyAsync(c->h_stage, dev, bytes, hipMemcpyDeviceToHost, c->stream), what);
  HIP_TRY(hipStreamSynchronize(c->stream), what);
  std::memcpy(host, c->h_stage, bytes);
  return BNR_OK;
}

// Grow-only zero-copy staging: pinned, non-coherent host memory mapped into
// the device's address space.  The kernels of the per-token host-slice
// entry points read their inputs from it and write their outputs into it,
// so such a call issues no copy commands.  What makes it safe without a
// stream synchronisation:
//  - outputs: a workgroup that wrote outputs into the staging makes them
//    host-visible before its completion word does -- signal_host waits for
//    the workgroup's stores and then stores the word with a system-scope
//    release, which writes this XCD's L2 back.  The rotated q and k of the
//    fused decode are written by split 0, which is not always the
//    workgroup that stores the word: split 0 issues a system-scope release
//    fence before its ticket, so they reach the host before the merging
//    workgroup (which takes the last ticket) stores the word.  The host
//    reads the staging only after every word of the call holds its
//    sequence number (host_wait_words), even though a kernel may still be
//    resident then;
//  - inputs: the host rewrites the staging only for the next call, after
//    every word of this one was set, i.e. after every workgroup of this
//    call has read its inputs.
// tests/test_gpu_host_words.py checks back-to-back host calls, each output
// checked on return.
int ensure_zc(bnr_ctx *c, size_t n) {
  if (c->h_zc_n >= n && c->h_zc) return BNR_OK;
  if (c->h_zc) {
    (void)hipStreamSynchronize(c->stream);
    (void)hipHostFree(c->h_zc);
    c->h_zc = c->d_zc = nullptr;
    c->h_zc_n = 0;
  }
  const size_t want = std::max<size_t>(n, 65536);
  HIP_TRY(hipHostMalloc((void **)&c->h_zc, want * sizeof(float),
                        hipHostMallocMapped | hipHostMallocNonCoherent),
          "zero-copy staging alloc");
  hipError_t e = hipHostGetDevicePointer((void **)&c->d_zc, c->h_zc, 0);
  if (e != hipSuccess) {
    (void)hipHostFree(c->h_zc);
    c->h_zc = c->d_zc = nullptr;
    return err_hip(e, "zero-copy staging map");
  }
  c->h_zc_n = want;
  return BNR_OK;
}

// Waits for the library's stream: a host-slice call returns with its
// outputs written.
int host_wait(bnr_ctx *c, const char *what) {
  HIP_TRY(hipStreamSynchronize(c->stream), what);
  return BNR_OK;
}

// Completion words: a host-slice call's kernel stores the call's sequence
// number into words 0..n-1 (one per workgroup that writes outputs) once its
// outputs are visible to the host.  The host thread watches them instead of
// sleeping in a stream synchronisation, whose wake-up costs several
// microseconds per call.
constexpr int kSignalWords = 4096;

// False when pinned, mapped memory cannot be had: the calls then wait with a
// stream synchronisation instead.
bool ensure_sig(bnr_ctx *c) {
  if (c->h_sig) return true;
  if (hipHostMalloc((void **)&c->h_sig, kSignalWords * sizeof(unsigned),
                    hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
    c->h_sig = nullptr;
    (void)hipGetLastError();
    return false;
  }
  std::memset(c->h_sig, 0, kSignalWords * sizeof(unsigned));
  if (hipHostGetDevicePointer((void **)&c->d_sig, c->h_sig, 0) != hipSuccess) {
    (void)hipHostFree(c->h_sig);
    c->h_sig = c->d_sig = nullptr;
    (void)hipGetLastError();
    return false;
  }
  return true;
}

// The next call's sequence number (never 0, the words' initial value).
unsigned next_seq(bnr_ctx *c) {
  if (++c->sig_seq == 0) c->sig_seq = 1;
  return c->sig_seq;
}

// Returns once words 0..n-1 hold seq.  The watch is bounded: after 2 ms
// (a kernel that faulted never stores) it falls back to synchronising the
// stream, which also reports any error.
int host_wait_words(bnr_ctx *c, int n, unsigned seq, const char *what) {
  const auto t0 = std::chrono::steady_clock::now();
  for (unsigned spins = 0;; ++spins) {
    int i = 0;
    while (i < n && __atomic_load_n(&c->h_sig[i], __ATOMIC_ACQUIRE) == seq) ++i;
    if (i == n) return BNR_OK;
    if ((spins & 255) == 255 &&
        std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(2000))
      return host_wait(c, what);
  }
}

// Grow-only, zero-filled ticket counters (kernels leave them zero).
int ensure_zeroed(unsigned **p, size_t *cap, size_t n) {
  if (*cap >= n && *p) return BNR_OK;
  if (*p) {
    (void)hipDeviceSynchronize();
    (void)hipFree(*p);
    *p = nullptr;
    *cap = 0;
  }
  size_t want = std::max<size_t>(n, 4096);
  HIP_TRY(hipMalloc((void **)p, want * sizeof(unsigned)), "counter alloc");
  HIP_TRY(hipMemset(*p, 0, want * sizeof(unsigned)), "counter clear");
  HIP_TRY(hipDeviceSynchronize(), "counter clear");
  *cap = want;
  return BNR_OK;
}

int ensure_ws(DecodeWs &w, size_t o_floats, size_t ml_n) {
  int st = ensure_buf(&w.ws_o, &w.ws_o_floats, o_floats, "workspace alloc");
  if (st) return st;
  if (w.ws_ml_n < ml_n || !w.ws_ml) {
    if (w.ws_ml) {
      (void)hipDeviceSynchronize();
      (void)hipFree(w.ws_ml);
      w.ws_ml = nullptr;
    }
    size_t want = std::max<size_t>(ml_n, 1024);
    HIP_TRY(hipMalloc((void **)&w.ws_ml, want * sizeof(float2)), "workspace alloc");
    w.ws_ml_n = want;
  }
  return BNR_OK;
}

void free_ws(DecodeWs &w) {
  if (w.ws_o) (void)hipFree(w.ws_o);
  if (w.ws_ml) (void)hipFree(w.ws_ml);
  if (w.counters) (void)hipFree(w.counters);
  if (w.acc) (void)hipFree(w.acc);
  if (w.scores) (void)hipFree(w.scores);
  if (w.rot) (void)hipFree(w.rot);
  w = DecodeWs{};
}

// The workspace of launches on stream s: the host-slice entry points run on
// the library's own stream, the device entry points on the caller's.
DecodeWs &ws_for(bnr_ctx *c, hipStream_t s) { return s == c->stream ? c->hws : c->dws; }

// The planner's choice for a prefill shape, remembered for the last 16
// shapes (planning replays the dispatch for every candidate).  Paired
// launches are planned for 4 q heads per kv head (two workgroups of the
// 16-query kernel per CU) unless forced.
PrefillPlanEntry plan_prefill_cached(bnr_ctx *c, int n_tokens, int start_pos, int n_kv, int group,
                                     long long cap) {
  const int pair_pref = c->pf_pair == 1 ? 1 : (c->pf_pair == -1 && group == 4 ? -1 : 0);
  for (const PrefillPlanEntry &e : c->pf_plans)
    if (e.n_tokens == n_tokens && e.start_pos == start_pos && e.n_kv == n_kv && e.cap == cap &&
        e.pair_pref == pair_pref)
      return e;
  PrefillPlanEntry e{n_tokens, start_pos, n_kv, pair_pref, cap, PrefillChoice{}, PairPlan{}};
  e.choice = plan_prefill_chunk(n_tokens, start_pos, n_kv, c->n_cu, c->pf_balanced, c->pf_q16,
                                cap, pair_pref, &e.pairs);
  if (c->pf_plans.size() >= 16) c->pf_plans.erase(c->pf_plans.begin());
  c->pf_plans.push_back(e);
  return e;
}

// RopeCache::new (bitnet-cpu/src/rope.rs:100-153) on the host: same f32
// formula, same libm, so the table is bit-identical to the reference's.
int build_table(bnr_ctx *c, size_t max_seq, size_t head_dim, float theta) {
  if (head_dim == 0 || head_dim % 2 != 0)
    return err_config(fmt("head_dim must be even and > 0, got %zu", head_dim));
  if (!(theta > 0.0f) || !std::isfinite(theta))
    return err_config("theta must be finite and > 0, got " + rust_f32(theta));
  const size_t half = head_dim / 2, n = max_seq * half;
  std::vector<float> hc(n), hs(n);
  for (size_t pos = 0; pos < max_seq; ++pos) {
    for (size_t i = 0; i < half; ++i) {
      volatile float exponent = -2.0f * (float)i / (float)head_dim;
      float freq = powf(theta, exponent);
      volatile float angle = (float)pos * freq;
      hc[pos * half + i] = cosf(angle);
      hs[pos * half + i] = sinf(angle);
    }
  }
  float *dc = nullptr, *ds = nullptr;
  HIP_TRY(hipMalloc((void **)&dc, std::max<size_t>(n, 1) * sizeof(float)), "rope table alloc");
  hipError_t e = hipMalloc((void **)&ds, std::max<size_t>(n, 1) * sizeof(float));
  if (e != hipSuccess) {
    (void)hipFree(dc);
    return err_hip(e, "rope table alloc");
  }
  e = hipMemcpy(dc, hc.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(ds, hs.data(), n * sizeof(float), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(dc);
    (void)hipFree(ds);
    return err_hip(e, "rope table upload");
  }
  if (c->d_cos) {
    (void)hipDeviceSynchronize();  // kernels in flight may still read the old table
    (void)hipFree(c->d_cos);
    (void)hipFree(c->d_sin);
  }
  c->d_cos = dc;
  c->d_sin = ds;
  c->tab_len = max_seq;
  c->tab_head_dim = head_dim;
  c->tab_theta = theta;
  c->tab_valid = true;
  return BNR_OK;
}

// CpuBackend::rope_embed's rebuild rule (bitnet-cpu/src/lib.rs:300-311).
int ensure_table(bnr_ctx *c, size_t position, size_t head_dim, float theta) {
  const bool reinit = !c->tab_valid || c->tab_head_dim != head_dim ||
                      std::fabs(c->tab_theta - theta) > 1e-3f || position >= c->tab_len;
  if (!reinit) return BNR_OK;
  size_t len = std::max<size_t>(position + 1, 4096);
  // A position past the end of a table of the same head_dim and exactly the
  // same theta grows it geometrically.  Entries depend on (position, i,
  // theta) only, so every value is the one the reference's max(position + 1,
  // 4096) table holds; only the rebuild on every call past the end is saved.
  // Any other theta rebuilds at max(position + 1, 4096), as the reference.
  if (c->tab_valid && c->tab_head_dim == head_dim && c->tab_theta == theta)
    len = std::max(len, 2 * c->tab_len);
  return build_table(c, len, head_dim, theta);
}

bool fast_shape(size_t n_heads, size_t n_kv, size_t head_dim) {
  if (head_dim != (size_t)kHeadDim || n_kv == 0 || n_kv > 64) return false;
  const size_t g = n_heads / n_kv;
  return g == 1 || g == 2 || g == 4;
}

// Split-K plan: rows per 16-lane row group (RPG) and passes per split.
// Small launches fit one workgroup per CU and have at most kMaxSplits
// splits per (sequence, kv head).
}  // namespace

void bnr::plan_decode(const DecodePlanConfig &cfg, const int *lens, int batch, int n_kv,
                      DecodeArgs &a) {
  const DecodePlanConfig *c = &cfg;
  int rpg = 1;
  long long wgs4 = 0;  // workgroups at 64 rows each
  for (int b = 0; b < batch; ++b) wgs4 += (lens[b] + 63) / 64;
  wgs4 *= n_kv;
  // Large launches: several workgroups per CU (batch > 1 and at least
  // large_wgs splits of 64 rows).  A single sequence never takes the large
  // path: its parallelism is the splits.  Merge modes: the reference merge
  // (default, decode_reg_kernel); for the deterministic decode_kernel, the
  // last workgroup's ticket merge (small launches) or a second kernel
  // (large ones).
  const bool large = batch > 1 && wgs4 >= c->large_wgs;
  const int mode = c->merge_mode >= 0 ? c->merge_mode : 2;
  a.merge_inline = mode != 0;
  a.merge_ref = mode >= 2;
  a.merge_det = mode == 3;
  const long long split_cost = c->split_cost >= 0 ? c->split_cost : 61;
  int passes = 1;
  if (a.merge_ref) {
    // Reference merge: the merge cost does not grow with the split count, so
    // a launch takes the fewest rows per split whose workgroups fit its
    // target: one round of one workgroup per CU (target_wgs) for a small
    // launch, eight workgroups per CU (two resident at rpg 4) for a large
    // one.  A split is a contiguous range of rows of one (sequence, kv head)
    // in passes of 4 * waves * rpg rows.
    const long long target = large ? 8LL * c->target_wgs : c->target_wgs;
    int max_len = 1;
    long long total = 0;
    for (int b = 0; b < batch; ++b) {
      max_len = std::max(max_len, lens[b]);
      total += lens[b];
    }
    int rows = c->ref_rows;
    if (rows <= 0) {
      // smallest rows in [lo, max_len] with sum_b ceil(lens[b] / rows) * n_kv
      // <= target (non-increasing in rows)
      auto fits = [&](int r) {
        long long wgs = 0;
        for (int b = 0; b < batch; ++b) wgs += (lens[b] + r - 1) / r;
        return wgs * n_kv <= target;
      };
      int lo = (int)std::max<long long>(1, (total * n_kv + target - 1) / target), hi = max_len;
      if (lo > hi) lo = hi;
      while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (fits(mid)) hi = mid;
        else lo = mid + 1;
      }
      rows = std::max(lo, 16);
    }
    rows = std::max(rows, (max_len + kMaxSplits - 1) / kMaxSplits);
    // Small launches run one workgroup per CU: 8 waves with up to 3 rows per
    // row group and pass, or 4 waves with up to 6 for sequences of at most
    // kRefWaves4Rows rows (graph-timed sweeps on MI355X, contexts
    // 512-32768).  Large ones run 4-wave workgroups with up to 3 rows per
    // row group while a split takes at most kLargeRpg3Rows rows (5 passes;
    // three workgroups resident per CU) and up to 4 beyond (two per CU, fewer
    // passes): 16-40 sequences of U[128, 4096) rows measured 3-11 % faster at
    // 3, 48 and 64 sequences 2-10 % slower.
    const int small_waves = c->ref_waves == 4 || c->ref_waves == 8
                                ? c->ref_waves
                                : (max_len <= kRefWaves4Rows ? 4 : 8);
    a.ref_waves = large ? 4 : small_waves;
    const int nrg = 4 * a.ref_waves;  // row groups of 16 lanes
    const int rpg_max = large ? (rows <= kLargeRpg3Rows ? 3 : 4) : a.ref_waves == 8 ? 3 : 6;
    const int r = c->force_rpg ? std::min(c->force_rpg, 6) : std::min(rpg_max, (rows + nrg - 1) / nrg);
    a.rpg = r;
    a.passes = (rows + nrg * r - 1) / (nrg * r);
    if (c->ref_rows <= 0) rows = std::max(nrg * r * a.passes, (max_len + kMaxSplits - 1) / kMaxSplits);
    a.rows_per_split = rows;
    a.batch = batch;
    a.split_off[0] = 0;
    a.max_splits = 1;
    for (int b = 0; b < batch; ++b) {
      const int ns = (lens[b] + rows - 1) / rows;
      a.split_off[b + 1] = a.split_off[b] + ns;
      a.max_splits = std::max(a.max_splits, ns);
    }
    return;
  }
  if (!large && !c->force_rpg) {
    // Small launches: among the splits of 16 * rpg * passes rows (rpg 1..8)
    // whose workgroups fit one per CU (at most target_wgs, by default the
    // CU count), the one with the lowest estimated time
    //   0.035 us per row of a workgroup + 0.061 us per split merged
    //   + 0.47 us per pass beyond the first,
    // a fit to graph-timed single-sequence launches on MI355X (contexts
    // 512-8192, rpg 1-8): rows cost the workgroup's loads and arithmetic,
    // splits cost the merge's loads, and each extra pass a load round trip.
    long long best = -1;
    rpg = 8;
    passes = 1;
    int max_len = 1;
    for (int b = 0; b < batch; ++b) max_len = std::max(max_len, lens[b]);
    const int p_max = std::max(c->min_passes, (max_len + 15) / 16);
    for (int p = c->min_passes; p <= p_max; ++p) {
      // No split of p passes beats `best` once its least cost (rpg 1, one
      // split) does not.
      if (best >= 0 && 35LL * 16 * p + split_cost + 474LL * (p - 1) >= best) break;
      for (int r = 1; r <= 8; ++r) {
        if (!a.merge_inline && (r & (r - 1))) continue;  // two-launch kernels: rpg 1, 2, 4, 8
        const int rows = 16 * r * p;
        long long wgs = 0;
        int splits = 0;
        for (int b = 0; b < batch; ++b) {
          const int ns = (lens[b] + rows - 1) / rows;
          wgs += ns;
          splits = std::max(splits, ns);
        }
        if (wgs * n_kv > c->target_wgs) continue;
        const long long cost = 35LL * rows + split_cost * splits + 474LL * (p - 1);
        if (best < 0 || cost < best) {
          best = cost;
          rpg = r;
          passes = p;
        }
      }
    }
    if (best < 0)  // more (sequence, kv head) pairs than target_wgs: one split each
      passes = std::max(c->min_passes, (max_len + 16 * 8 - 1) / (16 * 8));
  } else {
    rpg = c->force_rpg ? c->force_rpg : 4;
    if (!a.merge_inline && (rpg & (rpg - 1))) rpg = 4;  // two-launch kernels: rpg 1, 2, 4, 8
    int max_chunks = 0;
    for (int b = 0; b < batch; ++b) max_chunks = std::max(max_chunks, (lens[b] + 16 * rpg - 1) / (16 * rpg));
    passes = std::max(c->min_passes, (max_chunks + kMaxSplits - 1) / kMaxSplits);
    if (!large) {
      // A forced rpg: more passes per split rather than a second round of
      // workgroups (the RPG-6/8 kernels hold one workgroup per CU, the
      // others two or three).
      const long long resident = (long long)c->n_cu * (rpg >= 5 ? 1 : rpg >= 3 ? 2 : 3);
      auto wgs_at = [&](int p) {
        long long w = 0;
        for (int b = 0; b < batch; ++b) w += (lens[b] + 16 * rpg * p - 1) / (16 * rpg * p);
        return w * n_kv;
      };
      while (wgs_at(passes) > resident && passes < max_chunks) ++passes;
    }
  }
  const int rows = 16 * rpg * passes;
  a.rpg = rpg;
  a.passes = passes;
  a.rows_per_split = rows;
  a.batch = batch;
  a.split_off[0] = 0;
  a.max_splits = 1;
  for (int b = 0; b < batch; ++b) {
    const int ns = (lens[b] + rows - 1) / rows;
    a.split_off[b + 1] = a.split_off[b] + ns;
    a.max_splits = std::max(a.max_splits, ns);
  }
}

namespace {

// Launch the fast decode kernel over `batch` (<= kMaxBatchPerLaunch)
// sequences; a.{q,k_new,...,strides} are filled by the caller.
int run_decode(bnr_ctx *c, DecodeArgs &a, const int *positions, int batch, int n_kv, int group,
               size_t cap, hipStream_t s) {
  int lens[kMaxBatchPerLaunch];
  for (int b = 0; b < batch; ++b) {
    lens[b] = positions[b] + 1;
    a.positions[b] = positions[b];
  }
  const DecodePlanConfig pc{c->n_cu,       c->target_wgs, c->large_wgs,  c->force_rpg,
                            c->min_passes, c->merge_mode, c->split_cost, c->ref_rows,
                            c->ref_waves};
  plan_decode(pc, lens, batch, n_kv, a);
  a.n_kv = n_kv;
  a.group = group;
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)kHeadDim);
  // Size the workspace for the most splits any position below `cap` can
  // need, and tickets and accumulators for the largest batch of a launch,
  // so that later calls on the same caches -- including calls under HIP
  // graph capture -- never allocate.
  DecodeWs &w = ws_for(c, s);
  const size_t worst = std::min<size_t>(kMaxSplits, (cap + 15) / 16);
  const size_t splits = std::max<size_t>((size_t)a.split_off[batch], worst * (size_t)batch);
  int st = ensure_ws(w, splits * n_kv * group * kHeadDim, splits * n_kv * group);
  if (st) return st;
  const size_t heads = (size_t)std::max(batch, kMaxBatchPerLaunch) * n_kv;
  st = ensure_zeroed(&w.counters, &w.n_counters, heads * kCounterStride);
  if (st) return st;
  a.ws_o = w.ws_o;
  a.ws_ml = w.ws_ml;
  a.counters = w.counters;
  if (a.merge_ref) {
    st = ensure_zeroed(reinterpret_cast<unsigned **>(&w.acc), &w.acc_floats, heads * kAccStride);
    if (st) return st;
    a.acc = w.acc;
  }
  a.timeline = c->timeline;
  HIP_TRY(launch_decode(a, s), "decode launch");
  return BNR_OK;
}

int run_generic(bnr_ctx *c, const float *dq, const float *dk, const float *dv, long long kv_stride,
                float *dout, size_t n_heads, size_t n_kv, size_t head_dim, size_t cur_pos,
                hipStream_t s) {
  const size_t L = cur_pos + 1;
  // scores for every row of the cache (kv_stride / head_dim rows): later
  // calls on it never allocate
  const size_t rows = std::max(L, (size_t)kv_stride / head_dim);
  DecodeWs &w = ws_for(c, s);
  int st = ensure_buf(&w.scores, &w.scores_floats, n_heads * rows, "scratch alloc");
  if (st) return st;
  DecodeGenericArgs g{};
  g.q = dq;
  g.k_cache = dk;
  g.v_cache = dv;
  g.kv_stride = kv_stride;
  g.out = dout;
  g.scores = w.scores;
  g.n_heads = (int)n_heads;
  g.group = (int)(n_heads / n_kv);
  g.head_dim = (int)head_dim;
  g.L = (int)L;
  g.scale = 1.0f / sqrtf((float)head_dim);
  HIP_TRY(launch_decode_generic(g, s), "decode launch");
  return BNR_OK;
}

Mirror *find_mirror(bnr_ctx *c, const float *hk, size_t k_len, const float *hv, size_t v_len,
                    size_t n_kv, size_t head_dim) {
  for (auto it = c->mirrors.begin(); it != c->mirrors.end(); ++it) {
    if (it->hk == hk && it->hv == hv && it->k_len == k_len && it->v_len == v_len &&
        it->n_kv == n_kv && it->head_dim == head_dim) {
      c->mirrors.splice(c->mirrors.begin(), c->mirrors, it);
      return &c->mirrors.front();
    }
  }
  return nullptr;
}

}  // namespace

// ---------------------------------------------------------------------------
// Lifecycle
// ---------------------------------------------------------------------------
extern "C" const char *bnr_last_error(void) { return g_err.text.c_str(); }

extern "C" int bnr_last_error_parts(const char **first, const char **second) {
  if (first) *first = g_err.first.c_str();
  if (second) *second = g_err.second.c_str();
  return g_err.kind;
}

extern "C" uint32_t bnr_abi_version(void) { return (1u << 16) | 2u; }

extern "C" int bnr_create(int device_id, bnr_ctx **out) {
  if (!out) return err_backend("bnr_create: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    return err_device("no HIP device available");
  }
  if (device_id < 0 || device_id >= n) {
    return err_device(fmt("HIP device %d does not exist (%d present)", device_id, n));
  }
  hipDeviceProp_t prop;
  HIP_TRY(hipGetDeviceProperties(&prop, device_id), "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return err_device(fmt("HIP device %d is %s, this library is built for gfx950", device_id,
                          prop.gcnArchName));
  }
  DeviceGuard dg(device_id);
  bnr_ctx *c = new bnr_ctx();
  c->device = device_id;
  // The HIP runtime actually loaded (a process may hold PyTorch's bundled
  // runtime rather than the system one) goes into the name.
  int rt = 0, drv = 0;
  (void)hipRuntimeGetVersion(&rt);
  (void)hipDriverGetVersion(&drv);
  c->name = fmt("HIP (%s, %s, device %d; runtime %d, driver %d)", prop.name, prop.gcnArchName,
                device_id, rt, drv);
  e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return err_hip(e, "hipStreamCreate");
  }
  if (prop.multiProcessorCount > 0) c->n_cu = prop.multiProcessorCount;
  // The allocation-free entry point's scratch: resolved (and its merge state
  // zeroed) once per device; a failure here only disables that entry point.
  e = noalloc_scratch(device_id, c->stream, &c->noalloc);
  if (e != hipSuccess) {
    c->noalloc = nullptr;
    c->noalloc_err = std::string("no-alloc scratch setup failed: ") + hipGetErrorString(e);
  }
  c->target_wgs = c->n_cu;
  if (const char *v = std::getenv("BNR_DECODE_TARGET_WGS")) c->target_wgs = std::max(1, atoi(v));
  if (const char *v = std::getenv("BNR_DECODE_MERGE")) c->merge_mode = std::min(3, std::max(0, atoi(v)));
  if (const char *v = std::getenv("BNR_DECODE_SPLIT_COST")) c->split_cost = std::max(0, atoi(v));
  if (const char *v = std::getenv("BNR_DECODE_ROWS")) c->ref_rows = std::max(0, atoi(v));
  if (const char *v = std::getenv("BNR_DECODE_REF_WAVES")) c->ref_waves = atoi(v) == 8 ? 8 : 4;
  if (const char *v = std::getenv("BNR_DECODE_PASSES")) c->min_passes = std::min(64, std::max(1, atoi(v)));
  if (const char *v = std::getenv("BNR_DECODE_RPG")) {
    int r = atoi(v);
    if (r >= 1 && r <= 8) c->force_rpg = r;
  }
  if (const char *v = std::getenv("BNR_PREFILL_CHUNK_TILES"))
    c->pf_chunk_tiles = std::min(std::max(atoi(v), 1), kPrefillNoSplit);
  if (const char *v = std::getenv("BNR_PREFILL_PERSISTENT"))
    if (atoi(v) > 0) c->pf_mode = kPrefillQueue;
  if (const char *v = std::getenv("BNR_PREFILL_SK_WGS")) c->pf_sk_wgs = std::max(atoi(v), 0);
  if (const char *v = std::getenv("BNR_PREFILL_Q16")) c->pf_q16 = std::min(1, std::max(-1, atoi(v)));
  if (const char *v = std::getenv("BNR_PREFILL_BALANCED")) c->pf_balanced = std::min(1, std::max(-1, atoi(v)));
  if (const char *v = std::getenv("BNR_GEMV_NORM_MIN_WGS")) c->gemv_norm_min_wgs = std::max(1, atoi(v));
  if (const char *v = std::getenv("BNR_PREFILL_PAIR")) c->pf_pair = std::min(1, std::max(-1, atoi(v)));
  if (const char *v = std::getenv("BNR_PREFILL_MODE")) {
    const int m = atoi(v);
    if (m >= kPrefillGrid && m <= kPrefillAuto) c->pf_mode = m;
  }
  *out = c;
  return set_ok();
}

extern "C" void bnr_destroy(bnr_ctx *c) {
  if (!c) return;
  {
    std::lock_guard<std::mutex> lk(c->mu);
    DeviceGuard dg(c->device);
    (void)hipDeviceSynchronize();
    for (auto &m : c->mirrors) free_mirror(m);
    for (auto &m : c->weight_mirrors)
      if (m.dev) (void)hipFree(m.dev);
    if (c->d_bytes) (void)hipFree(c->d_bytes);
    if (c->h_stage) (void)hipHostFree(c->h_stage);
    if (c->h_zc) (void)hipHostFree(c->h_zc);
    if (c->h_sig) (void)hipHostFree(c->h_sig);
    float *bufs[] = {c->d_cos, c->d_sin, c->d_q, c->d_out, c->pf_ws};
    for (float *p : bufs)
      if (p) (void)hipFree(p);
    free_ws(c->hws);
    free_ws(c->dws);
    if (c->pf_counters) (void)hipFree(c->pf_counters);
    if (c->pf_queue) (void)hipFree(c->pf_queue);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    noalloc_release(c->device, c);
  }
  delete c;
}

extern "C" const char *bnr_device_name(const bnr_ctx *c) { return c ? c->name.c_str() : ""; }

// ---------------------------------------------------------------------------
// Trait-shaped host entry points
// ---------------------------------------------------------------------------
extern "C" int bnr_rope_embed(bnr_ctx *c, float *q, size_t q_len, float *k, size_t k_len,
                              size_t position, size_t head_dim, size_t n_heads,
                              size_t n_kv_heads, float theta) {
  if (!c) return err_backend("context is NULL");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  // CpuBackend::rope_embed: table policy first (lib.rs:299-311), then
  // apply_rope_cached's length checks (rope.rs:324-337).
  int st = ensure_table(c, position, head_dim, theta);
  if (st) return st;
  const size_t hd = c->tab_head_dim;
  if (q_len != n_heads * hd)
    return err_shape(fmt("q.len() == %zu * %zu = %zu", n_heads, hd, n_heads * hd),
                     fmt("q.len() = %zu", q_len));
  if (k_len != n_kv_heads * hd)
    return err_shape(fmt("k.len() == %zu * %zu = %zu", n_kv_heads, hd, n_kv_heads * hd),
                     fmt("k.len() = %zu", k_len));
  if (q_len + k_len == 0) return set_ok();
  if ((q_len && !q) || (k_len && !k)) return err_backend("rope_embed: NULL slice");
  // q and k rotate in place in the zero-copy staging: [q | k], k 16-byte
  // aligned.
  const size_t qs = round4(q_len), total = qs + k_len;
  st = ensure_zc(c, total);
  if (st) return st;
  float *h = c->h_zc;
  if (q_len) std::memcpy(h, q, q_len * sizeof(float));
  if (k_len) std::memcpy(h + qs, k, k_len * sizeof(float));
  RopeAppendArgs a{};
  a.q = c->d_zc;
  a.k = c->d_zc + qs;
  a.n_tokens = 1;
  a.start_pos = (int)position;
  a.n_heads = (int)n_heads;
  a.n_kv = (int)n_kv_heads;
  a.head_dim = (int)hd;
  a.cos_tab = c->d_cos;
  a.sin_tab = c->d_sin;
  const long long words = rope_append_blocks(a);
  const bool watch = words <= kSignalWords && ensure_sig(c);
  if (watch) {
    a.done = c->d_sig;
    a.seq = next_seq(c);
  }
  HIP_TRY(launch_rope_append(a, c->stream), "rope launch");
  st = watch ? host_wait_words(c, (int)words, a.seq, "rope_embed") : host_wait(c, "rope_embed");
  if (st) return st;
  if (q_len) std::memcpy(q, h, q_len * sizeof(float));
  if (k_len) std::memcpy(k, h + qs, k_len * sizeof(float));
  return set_ok();
}

extern "C" int bnr_masked_attention(bnr_ctx *c, const float *q, size_t q_len,
                                    const float *k_cache, size_t k_len, const float *v_cache,
                                    size_t v_len, float *output, size_t out_len, size_t n_heads,
                                    size_t n_kv_heads, size_t head_dim, size_t cur_pos) {
  if (!c) return err_backend("context is NULL");
  // Validation order of attention::masked_attention (attention.rs:109-161).
  if (head_dim == 0) return err_shape("head_dim > 0", "head_dim = 0");
  if (n_kv_heads == 0) return err_config("n_kv_heads must be > 0");
  if (n_heads == 0) return err_config("n_heads must be > 0");
  if (n_heads % n_kv_heads != 0)
    return err_config(fmt("n_heads (%zu) must be divisible by n_kv_heads (%zu)", n_heads, n_kv_heads));
  const size_t seq_len = cur_pos + 1;
  const size_t head_stride = k_len / n_kv_heads;
  const size_t required = n_kv_heads * head_stride;
  const size_t q_expected = n_heads * head_dim;
  if (q_len != q_expected)
    return err_shape(fmt("q.len() == n_heads * head_dim = %zu * %zu = %zu", n_heads, head_dim, q_expected),
                     fmt("q.len() = %zu", q_len));
  if (k_len < required)
    return err_shape(fmt("k_cache.len() >= %zu", required), fmt("k_cache.len() = %zu", k_len));
  if (v_len < required)
    return err_shape(fmt("v_cache.len() >= %zu", required), fmt("v_cache.len() = %zu", v_len));
  if (head_stride < seq_len * head_dim)
    return err_shape(fmt("per-head cache stride >= %zu", seq_len * head_dim),
                     fmt("per-head cache stride = %zu", head_stride));
  if (out_len != q_expected)
    return err_shape(fmt("output.len() == n_heads * head_dim = %zu", q_expected),
                     fmt("output.len() = %zu", out_len));
  if (!q || !k_cache || !v_cache || !output) return err_backend("masked_attention: NULL slice");

  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);

  // ---- HBM mirror of this layer's cache ----
  const size_t rows = head_stride / head_dim;  // >= seq_len by the checks above
  Mirror *m = find_mirror(c, k_cache, k_len, v_cache, v_len, n_kv_heads, head_dim);
  if (!m) {
    if (c->mirrors.size() >= kMaxMirrors) {
      (void)hipStreamSynchronize(c->stream);
      free_mirror(c->mirrors.back());
      c->mirrors.pop_back();
    }
    Mirror nm;
    nm.hk = k_cache;
    nm.hv = v_cache;
    nm.k_len = k_len;
    nm.v_len = v_len;
    nm.n_kv = n_kv_heads;
    nm.head_dim = head_dim;
    nm.rows = rows;
    const size_t bytes = n_kv_heads * rows * head_dim * sizeof(float);
    HIP_TRY(hipMalloc((void **)&nm.dk, bytes), "mirror alloc");
    hipError_t e = hipMalloc((void **)&nm.dv, bytes);
    if (e != hipSuccess) {
      (void)hipFree(nm.dk);
      return err_hip(e, "mirror alloc");
    }
    c->mirrors.push_front(nm);
    m = &c->mirrors.front();
  }
  size_t r0 = 0;
  if (c->mirror_mode == BNR_MIRROR_INCREMENTAL && m->synced == cur_pos) {
    kv_probe(k_cache, v_cache, n_kv_heads, head_stride, head_dim, cur_pos, c->probe_now);
    if (c->probe_now.size() == m->probe.size() &&
        std::memcmp(c->probe_now.data(), m->probe.data(), m->probe.size() * sizeof(float)) == 0)
      r0 = cur_pos;
  }
  if (r0 == cur_pos && cur_pos > 0 && fast_shape(n_heads, n_kv_heads, head_dim)) {
    // One new row: the decode kernel reads q and row cur_pos of every kv
    // head from the zero-copy staging, appends the row to the mirror itself
    // (fused append, no rotation) and writes the output back into the
    // staging: [q | k row | v row | out].
    const size_t rs = n_kv_heads * head_dim, in_n = q_len + 2 * rs;
    int st = ensure_zc(c, in_n + out_len);
    if (st) return st;
    float *h = c->h_zc, *d = c->d_zc;
    std::memcpy(h, q, q_len * sizeof(float));
    for (size_t kh = 0; kh < n_kv_heads; ++kh) {
      const size_t src = kh * head_stride + cur_pos * head_dim;
      std::memcpy(h + q_len + kh * head_dim, k_cache + src, head_dim * sizeof(float));
      std::memcpy(h + q_len + rs + kh * head_dim, v_cache + src, head_dim * sizeof(float));
    }
    m->synced = 0;  // unknown until the launch succeeds
    DecodeArgs a{};
    a.q = d;
    a.k_new = d + q_len;
    a.v_new = d + q_len + rs;
    a.k_cache = m->dk;
    a.v_cache = m->dv;
    a.kv_stride = (long long)(m->rows * head_dim);
    a.out = d + in_n;
    const bool sig = (int)n_kv_heads <= kSignalWords && ensure_sig(c);
    if (sig) {
      a.done = c->d_sig;  // set by the reference-merge kernel (the launch checks below)
      a.seq = next_seq(c);
    }
    const int p = (int)cur_pos;
    st = run_decode(c, a, &p, 1, (int)n_kv_heads, (int)(n_heads / n_kv_heads), m->rows, c->stream);
    if (st) return st;
    st = sig && a.merge_ref && a.group <= 4
             ? host_wait_words(c, (int)n_kv_heads, a.seq, "masked_attention")
             : host_wait(c, "masked_attention");
    if (st) return st;
    std::memcpy(output, h + in_n, out_len * sizeof(float));
    m->synced = seq_len;
    kv_probe(k_cache, v_cache, n_kv_heads, head_stride, head_dim, seq_len, m->probe);
    return set_ok();
  }
  const size_t dpitch = m->rows * head_dim * sizeof(float);
  const size_t spitch = head_stride * sizeof(float);
  const size_t width = (seq_len - r0) * head_dim * sizeof(float);
  m->synced = 0;  // unknown until both copies succeed
  HIP_TRY(hipMemcpy2DAsync(m->dk + r0 * head_dim, dpitch, k_cache + r0 * head_dim, spitch, width,
                           n_kv_heads, hipMemcpyHostToDevice, c->stream),
          "mirror upload k");
  HIP_TRY(hipMemcpy2DAsync(m->dv + r0 * head_dim, dpitch, v_cache + r0 * head_dim, spitch, width,
                           n_kv_heads, hipMemcpyHostToDevice, c->stream),
          "mirror upload v");
  m->synced = seq_len;
  kv_probe(k_cache, v_cache, n_kv_heads, head_stride, head_dim, seq_len, m->probe);

  int st = ensure_buf(&c->d_q, &c->d_q_n, q_len, "staging alloc");
  if (st) return st;
  st = ensure_buf(&c->d_out, &c->d_out_n, out_len, "staging alloc");
  if (st) return st;
  HIP_TRY(hipMemcpyAsync(c->d_q, q, q_len * 4, hipMemcpyHostToDevice, c->stream), "upload q");
  const long long kv_stride = (long long)(m->rows * head_dim);
  if (fast_shape(n_heads, n_kv_heads, head_dim)) {
    DecodeArgs a{};
    a.q = c->d_q;
    a.k_cache = m->dk;
    a.v_cache = m->dv;
    a.kv_stride = kv_stride;
    a.out = c->d_out;
    const int p = (int)cur_pos;
    st = run_decode(c, a, &p, 1, (int)n_kv_heads, (int)(n_heads / n_kv_heads), m->rows, c->stream);
  } else {
    st = run_generic(c, c->d_q, m->dk, m->dv, kv_stride, c->d_out, n_heads, n_kv_heads, head_dim,
                     cur_pos, c->stream);
  }
  if (st) {
    m->synced = 0;
    return st;
  }
  HIP_TRY(hipMemcpyAsync(output, c->d_out, out_len * 4, hipMemcpyDeviceToHost, c->stream), "download out");
  hipError_t e = hipStreamSynchronize(c->stream);
  if (e != hipSuccess) {
    m->synced = 0;
    return err_hip(e, "masked_attention");
  }
  return set_ok();
}

extern "C" int bnr_set_deterministic(bnr_ctx *c, int on) {
  if (!c) return err_backend("context is NULL");
  std::lock_guard<std::mutex> lk(c->mu);
  c->merge_mode = on ? 3 : -1;
  return set_ok();
}

extern "C" int bnr_set_mirror_mode(bnr_ctx *c, int mode) {
  if (!c) return err_backend("context is NULL");
  if (mode != BNR_MIRROR_INCREMENTAL && mode != BNR_MIRROR_FULL)
    return err_config(fmt("unknown mirror mode %d", mode));
  std::lock_guard<std::mutex> lk(c->mu);
  c->mirror_mode = mode;
  return set_ok();
}

extern "C" int bnr_mirror_invalidate(bnr_ctx *c) {
  if (!c) return err_backend("context is NULL");
  std::lock_guard<std::mutex> lk(c->mu);
  for (auto &m : c->mirrors) m.synced = 0;
  if (!c->weight_mirrors.empty()) {
    DeviceGuard dg(c->device);
    (void)hipStreamSynchronize(c->stream);
    for (auto &m : c->weight_mirrors)
      if (m.dev) (void)hipFree(m.dev);
    c->weight_mirrors.clear();
  }
  return set_ok();
}

// ---------------------------------------------------------------------------
// W2A8 ternary GEMV
// ---------------------------------------------------------------------------
namespace {

// Checks of gemv::ternary_gemv_quantised (bitnet-cpu/src/gemv.rs:260-295),
// in its order, for the lengths that are given (SIZE_MAX: not checked).
int check_gemv(size_t weight_len, float weight_scale, size_t act_len, float act_absmax,
               size_t out_len, size_t out_features, size_t in_features) {
  const size_t packed_cols = (in_features + 3) / 4;
  if (packed_cols != 0 && out_features > SIZE_MAX / packed_cols)
    return err_shape("weight size fits usize", "overflow");
  const size_t expected = out_features * packed_cols;
  if (weight_len != SIZE_MAX && weight_len != expected)
    return err_shape(fmt("weight_packed.len() == %zu * ceil(%zu/4) = %zu", out_features,
                         in_features, expected),
                     fmt("weight_packed.len() == %zu", weight_len));
  if (act_len != SIZE_MAX && act_len != in_features)
    return err_shape(fmt("activation.len() == %zu", in_features),
                     fmt("activation.len() == %zu", act_len));
  if (out_len != SIZE_MAX && out_len != out_features)
    return err_shape(fmt("output.len() == %zu", out_features), fmt("output.len() == %zu", out_len));
  if (weight_scale <= 0.0f || !std::isfinite(weight_scale))
    return err_quant("weight_scale must be finite > 0, got " + rust_f32(weight_scale));
  if (act_absmax <= 0.0f || !std::isfinite(act_absmax))
    return err_quant("act_scale must be finite > 0, got " + rust_f32(act_absmax));
  if (out_features > (size_t)INT32_MAX || in_features > (size_t)INT32_MAX)
    return err_backend("ternary_gemv_preq: dimensions beyond 2^31 are not supported");
  return BNR_OK;
}

int run_gemv(const uint8_t *w, float weight_scale, const int8_t *act, float act_absmax, float *out,
             size_t out_features, size_t in_features, hipStream_t s) {
  TernaryGemvArgs a{};
  a.weight = w;
  a.act = act;
  a.out = out;
  a.packed_cols = (long long)((in_features + 3) / 4);
  a.out_features = (int)out_features;
  a.in_features = (int)in_features;
  // combined_scale = weight_scale * act_scale / 127.0 (gemv.rs:297), f32, left to right
  volatile float ws_as = weight_scale * act_absmax;
  a.scale = ws_as / 127.0f;
  const bool vec = a.packed_cols % 16 == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)act % 16) == 0;
  HIP_TRY(launch_ternary_gemv(a, vec, s), "ternary_gemv launch");
  return BNR_OK;
}

}  // namespace

// HBM copy of immutable host bytes (weights, scales), most recently used
// first; *dev receives the device address.  Caller holds c->mu.
int mirror_bytes(bnr_ctx *c, const void *host_p, size_t len, const uint8_t **dev) {
  const uint8_t *host = (const uint8_t *)host_p;
  uint8_t print[kFingerprint];
  fingerprint(host, len, print);
  auto it = c->weight_mirrors.begin();
  for (; it != c->weight_mirrors.end(); ++it)
    if (it->host == host && it->len == len) break;
  if (it != c->weight_mirrors.end() && std::memcmp(it->print, print, kFingerprint) != 0) {
    (void)hipStreamSynchronize(c->stream);  // different contents at the same address
    (void)hipFree(it->dev);
    c->weight_mirrors.erase(it);
    it = c->weight_mirrors.end();
  }
  if (it != c->weight_mirrors.end()) {
    c->weight_mirrors.splice(c->weight_mirrors.begin(), c->weight_mirrors, it);
  } else {
    if (c->weight_mirrors.size() >= kMaxWeightMirrors) {
      (void)hipStreamSynchronize(c->stream);
      (void)hipFree(c->weight_mirrors.back().dev);
      c->weight_mirrors.pop_back();
    }
    WeightMirror m;
    m.host = host;
    m.len = len;
    std::memcpy(m.print, print, kFingerprint);
    HIP_TRY(hipMalloc((void **)&m.dev, len), "weight mirror alloc");
    hipError_t e = hipMemcpyAsync(m.dev, host, len, hipMemcpyHostToDevice, c->stream);
    if (e != hipSuccess) {
      (void)hipFree(m.dev);
      return err_hip(e, "weight upload");
    }
    c->weight_mirrors.push_front(m);
  }
  *dev = c->weight_mirrors.front().dev;
  return BNR_OK;
}

extern "C" int bnr_ternary_gemv_preq(bnr_ctx *c, const uint8_t *weight_packed, size_t weight_len,
                                     float weight_scale, const int8_t *activation_q,
                                     size_t act_len, float act_absmax, float *output,
                                     size_t out_len, size_t out_features, size_t in_features) {
  if (!c) return err_backend("context is NULL");
  int st = check_gemv(weight_len, weight_scale, act_len, act_absmax, out_len, out_features,
                      in_features);
  if (st) return st;
  if (out_features == 0) return set_ok();
  if ((weight_len && !weight_packed) || (act_len && !activation_q) || !output)
    return err_backend("ternary_gemv_preq: NULL slice");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  const uint8_t *dw = nullptr;
  if (weight_len) {
    st = mirror_bytes(c, weight_packed, weight_len, &dw);
    if (st) return st;
  }
  if (c->d_bytes_n < std::max<size_t>(in_features, 16)) {
    if (c->d_bytes) {
      (void)hipStreamSynchronize(c->stream);
      (void)hipFree(c->d_bytes);
      c->d_bytes = nullptr;
      c->d_bytes_n = 0;
    }
    const size_t want = std::max<size_t>(in_features, 4096);
    HIP_TRY(hipMalloc((void **)&c->d_bytes, want), "staging alloc");
    c->d_bytes_n = want;
  }
  st = ensure_buf(&c->d_out, &c->d_out_n, out_features, "staging alloc");
  if (st) return st;
  if (in_features) {
    st = put_host(c, c->d_bytes, {{activation_q, in_features}}, "upload activation");
    if (st) return st;
  }
  st = run_gemv(dw, weight_scale, (const int8_t *)c->d_bytes, act_absmax, c->d_out, out_features,
                in_features, c->stream);
  if (st) return st;
  st = get_host(c, output, c->d_out, out_features * 4, "ternary_gemv_preq");
  return st ? st : set_ok();
}

// ---------------------------------------------------------------------------
// Device entry points
// ---------------------------------------------------------------------------
namespace {

int check_heads(size_t n_heads, size_t n_kv, size_t head_dim) {
  if (head_dim == 0) return err_shape("head_dim > 0", "head_dim = 0");
  if (n_kv == 0) return err_config("n_kv_heads must be > 0");
  if (n_heads == 0) return err_config("n_heads must be > 0");
  if (n_heads % n_kv != 0)
    return err_config(fmt("n_heads (%zu) must be divisible by n_kv_heads (%zu)", n_heads, n_kv));
  return BNR_OK;
}

int check_rope(size_t head_dim, float theta) {
  if (head_dim == 0 || head_dim % 2 != 0)
    return err_config(fmt("head_dim must be even and > 0, got %zu", head_dim));
  if (!(theta > 0.0f) || !std::isfinite(theta))
    return err_config("theta must be finite and > 0, got " + rust_f32(theta));
  return BNR_OK;
}

int check_rows(size_t last_pos, size_t cap) {
  if (last_pos >= cap)
    return err_shape(fmt("position < max_seq (%zu)", cap), fmt("position = %zu", last_pos));
  return BNR_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

int launch_rope_append_dev(bnr_ctx *c, float *q, float *k, const float *v, size_t n_tokens,
                           size_t start_pos, size_t n_heads, size_t n_kv, size_t head_dim,
                           float *k_cache, float *v_cache, size_t cap, hipStream_t s) {
  RopeAppendArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.n_tokens = (int)n_tokens;
  a.start_pos = (int)start_pos;
  a.n_heads = (int)n_heads;
  a.n_kv = (int)n_kv;
  a.head_dim = (int)head_dim;
  a.cos_tab = c->d_cos;
  a.sin_tab = c->d_sin;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.kv_stride = (long long)(cap * head_dim);
  HIP_TRY(launch_rope_append(a, s), "rope/append launch");
  return BNR_OK;
}

}  // namespace

extern "C" int bnr_dev_rope_append(bnr_ctx *c, float *q, float *k, const float *v,
                                   size_t n_tokens, size_t start_pos, size_t n_heads,
                                   size_t n_kv_heads, size_t head_dim, float theta,
                                   float *k_cache, float *v_cache, size_t cap, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rope(head_dim, theta);
  if (st) return st;
  if (n_tokens == 0) return set_ok();
  st = check_rows(start_pos + n_tokens - 1, cap);
  if (st) return st;
  if (!q || !k || !v || !k_cache || !v_cache) return err_backend("rope_append: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  // The table covers every row of the cache, so later calls on it (also
  // under HIP graph capture) never rebuild it.
  st = ensure_table(c, std::max(start_pos + n_tokens, cap) - 1, head_dim, theta);
  if (st) return st;
  st = launch_rope_append_dev(c, q, k, v, n_tokens, start_pos, n_heads, n_kv_heads, head_dim,
                              k_cache, v_cache, cap, (hipStream_t)stream);
  return st ? st : set_ok();
}

extern "C" int bnr_dev_decode_attention(bnr_ctx *c, const float *q, const float *k_cache,
                                        const float *v_cache, size_t cap, float *out,
                                        size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                        size_t cur_pos, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rows(cur_pos, cap);
  if (st) return st;
  if (!q || !k_cache || !v_cache || !out) return err_backend("decode_attention: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  hipStream_t s = (hipStream_t)stream;
  const long long kv_stride = (long long)(cap * head_dim);
  if (fast_shape(n_heads, n_kv_heads, head_dim) && aligned16(q) && aligned16(k_cache) &&
      aligned16(v_cache)) {
    DecodeArgs a{};
    a.q = q;
    a.k_cache = const_cast<float *>(k_cache);
    a.v_cache = const_cast<float *>(v_cache);
    a.kv_stride = kv_stride;
    a.out = out;
    const int p = (int)cur_pos;
    st = run_decode(c, a, &p, 1, (int)n_kv_heads, (int)(n_heads / n_kv_heads), cap, s);
  } else {
    st = run_generic(c, q, k_cache, v_cache, kv_stride, out, n_heads, n_kv_heads, head_dim, cur_pos, s);
  }
  return st ? st : set_ok();
}

extern "C" int bnr_dev_stream_read(bnr_ctx *c, const void *a, size_t a_bytes, const void *b,
                                   size_t b_bytes, void *stream) {
  if (!c) return err_backend("context is NULL");
  if ((a_bytes && !a) || (b_bytes && !b)) return err_backend("stream_read: NULL pointer");
  if (a_bytes % 16 || b_bytes % 16 || !aligned16(a) || !aligned16(b))
    return err_shape("16-byte aligned ranges of whole 16-byte words", "an unaligned range");
  DeviceGuard dg(c->device);
  HIP_TRY(launch_stream_read(a, (long long)a_bytes, b, (long long)b_bytes, (hipStream_t)stream),
          "stream read launch");
  return set_ok();
}

#if defined(BNR_TIMELINE)
// Measurement builds only (not in the public header): the next decode and
// grid-mapped prefill launches of this context store kTimelineStamps stamps
// per workgroup at `stamps` (device memory, 8 bytes each, one slot per
// workgroup of the grid; null: none).
extern "C" int bnr_debug_decode_timeline(bnr_ctx *c, void *stamps) {
  if (!c) return err_backend("context is NULL");
  c->timeline = static_cast<unsigned long long *>(stamps);
  return set_ok();
}

namespace bnr {
hipError_t launch_rt_probe(unsigned *buf, int n, int mode, unsigned long long *out, hipStream_t s);
hipError_t launch_empty(int wgs, int threads, int mode, unsigned *buf, hipStream_t s);
}  // namespace bnr

// Round trips of device-scope operations (one lane, n dependent operations
// of the given mode on buf, at least 512 bytes of zeroed device memory;
// out[0] = elapsed 100 MHz ticks).
extern "C" int bnr_debug_rt_probe(bnr_ctx *c, void *buf, int n, int mode, void *out, void *stream) {
  if (!c || !buf || !out || n < 1 || mode < 0 || mode > 3) return err_backend("rt_probe: bad arguments");
  DeviceGuard dg(c->device);
  HIP_TRY(launch_rt_probe(static_cast<unsigned *>(buf), n, mode,
                          static_cast<unsigned long long *>(out), (hipStream_t)stream),
          "rt_probe launch");
  return set_ok();
}

// An empty launch of wgs workgroups of `threads` threads (at most 512);
// mode 0 bare, 1 with the decode's argument block, 2 with 64 KB of LDS,
// 3 with both; 4-7: one word per workgroup written into buf (at least 64 KB
// of device memory): a plain store, a non-temporal store, a device-scope
// atomic add, a system-scope store; 8: the argument block, 64 KB of LDS
// and 160 VGPRs (the 8-wave decode kernel's footprint).
extern "C" int bnr_debug_empty_launch(bnr_ctx *c, int wgs, int threads, int mode, void *buf,
                                      void *stream) {
  if (!c || wgs < 1 || threads < 1 || threads > 512 || mode < 0 || mode > 8 || (mode >= 4 && mode <= 7 && !buf))
    return err_backend("empty_launch: bad arguments");
  DeviceGuard dg(c->device);
  HIP_TRY(launch_empty(wgs, threads, mode, static_cast<unsigned *>(buf), (hipStream_t)stream),
          "empty launch");
  return set_ok();
}
#endif

extern "C" int bnr_dev_stream_read_shape(bnr_ctx *c, const void *a, size_t a_bytes, const void *b,
                                         size_t b_bytes, int threads, int loads_per_lane,
                                         int nontemporal, void *stream) {
  if (!c) return err_backend("context is NULL");
  if ((a_bytes && !a) || (b_bytes && !b)) return err_backend("stream_read: NULL pointer");
  if (a_bytes % 16 || b_bytes % 16 || !aligned16(a) || !aligned16(b))
    return err_shape("16-byte aligned ranges of whole 16-byte words", "an unaligned range");
  if (threads < 64 || threads > 1024 || threads % 64)
    return err_config(fmt("threads must be a multiple of 64 in 64..=1024, got %d", threads));
  if (loads_per_lane != 1 && loads_per_lane != 2 && loads_per_lane != 4 && loads_per_lane != 8 &&
      loads_per_lane != 16)
    return err_config(fmt("loads_per_lane must be 1, 2, 4, 8 or 16, got %d", loads_per_lane));
  DeviceGuard dg(c->device);
  HIP_TRY(launch_stream_read_shape(a, (long long)a_bytes, b, (long long)b_bytes, threads,
                                   loads_per_lane, nontemporal != 0, (hipStream_t)stream),
          "stream read launch");
  return set_ok();
}

extern "C" int bnr_dev_decode_attention_noalloc(bnr_ctx *c, const float *q, const float *k_cache,
                                                const float *v_cache, size_t cap, float *out,
                                                size_t n_heads, size_t n_kv_heads,
                                                size_t head_dim, size_t cur_pos, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rows(cur_pos, cap);
  if (st) return st;
  if (!q || !k_cache || !v_cache || !out) return err_backend("decode_attention_noalloc: NULL pointer");
  if (!fast_shape(n_heads, n_kv_heads, head_dim))
    return err_config(fmt("decode_attention_noalloc needs head_dim %d and n_heads/n_kv_heads in "
                          "{1,2,4}, got head_dim %zu, n_heads %zu, n_kv_heads %zu",
                          kHeadDim, head_dim, n_heads, n_kv_heads));
  if (n_heads > (size_t)kNoAllocMaxHeads)
    return err_config(fmt("decode_attention_noalloc holds at most %d query heads, got %zu",
                          kNoAllocMaxHeads, n_heads));
  if (!(aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out)))
    return err_shape("16-byte aligned device pointers", "an unaligned pointer");
  if (cur_pos >= (size_t)INT32_MAX)
    return err_shape(fmt("cur_pos < %d", INT32_MAX), fmt("cur_pos = %zu", cur_pos));
  std::lock_guard<std::mutex> lk(c->mu);
  if (!c->noalloc) return err_backend(c->noalloc_err.empty() ? "no-alloc scratch unavailable" : c->noalloc_err);
  if (!noalloc_claim(c->device, c, stream))
    return err_backend(fmt("decode_attention_noalloc: GPU %d's scratch is held by another context "
                           "or stream (launches from two could overlap on the GPU and race); "
                           "use one context and one stream, or destroy the other context first",
                           c->device));
  DeviceGuard dg(c->device);
  DecodeArgs a{};
  a.q = q;
  a.k_cache = const_cast<float *>(k_cache);
  a.v_cache = const_cast<float *>(v_cache);
  a.kv_stride = (long long)(cap * head_dim);
  a.out = out;
  const int lens[1] = {(int)cur_pos + 1};
  a.positions[0] = (int)cur_pos;
  // Always the reference merge: its state fits the scratch for any context.
  const DecodePlanConfig pc{c->n_cu, c->target_wgs, c->large_wgs, c->force_rpg, c->min_passes,
                            2,       c->split_cost, c->ref_rows, c->ref_waves};
  plan_decode(pc, lens, 1, (int)n_kv_heads, a);
  if (a.max_splits > kMaxSplits) return err_backend("decode_attention_noalloc: too many splits");
  a.n_kv = (int)n_kv_heads;
  a.group = (int)(n_heads / n_kv_heads);
  a.scale_log2 = 1.4426950408889634f / sqrtf((float)kHeadDim);
  char *base = static_cast<char *>(c->noalloc);
  a.acc = reinterpret_cast<float *>(base);
  a.counters = reinterpret_cast<unsigned *>(base + kNoAllocAccBytes);
  a.ws_ml = reinterpret_cast<float2 *>(base + kNoAllocZeroBytes);
  a.ws_o = reinterpret_cast<float *>(base + kNoAllocZeroBytes + kNoAllocMlBytes);
  HIP_TRY(launch_decode(a, (hipStream_t)stream), "decode launch");
  return set_ok();
}

namespace {

// bnr_dev_decode_step after validation; the caller holds c->mu.
// done/seq (host-slice calls): completion words for the reference-merge
// kernel; *signals tells whether the launch stores them.
int decode_step_locked(bnr_ctx *c, const float *q, const float *k, const float *v,
                       size_t position, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                       float theta, float *k_cache, float *v_cache, size_t cap, float *out,
                       float *q_rot, float *k_rot, hipStream_t s, unsigned *done = nullptr,
                       unsigned seq = 0, bool *signals = nullptr) {
  if (signals) *signals = false;
  DeviceGuard dg(c->device);
  // The table covers every row of the cache (no rebuild on later calls).
  int st = ensure_table(c, std::max(position + 1, cap) - 1, head_dim, theta);
  if (st) return st;
  const long long kv_stride = (long long)(cap * head_dim);
  const bool al = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(k_cache) &&
                  aligned16(v_cache) && (!q_rot || aligned16(q_rot)) && (!k_rot || aligned16(k_rot));
  if (fast_shape(n_heads, n_kv_heads, head_dim) && al) {
    DecodeArgs a{};
    a.q = q;
    a.k_new = k;
    a.v_new = v;
    a.k_cache = k_cache;
    a.v_cache = v_cache;
    a.kv_stride = kv_stride;
    a.out = out;
    a.q_rot = q_rot;
    a.k_rot = k_rot;
    a.cos_tab = c->d_cos;
    a.sin_tab = c->d_sin;
    a.done = done;
    a.seq = seq;
    const int p = (int)position;
    st = run_decode(c, a, &p, 1, (int)n_kv_heads, (int)(n_heads / n_kv_heads), cap, s);
    if (!st && signals) *signals = done && a.merge_ref && a.group <= 4;
    return st ? st : set_ok();
  }
  // Any other shape: rotate copies, append, then the generic kernel.
  const size_t qn = n_heads * head_dim, kn = n_kv_heads * head_dim;
  float *qw = q_rot, *kw = k_rot;
  DecodeWs &w = ws_for(c, s);
  st = ensure_buf(&w.rot, &w.rot_floats, qn + kn, "staging alloc");
  if (st) return st;
  if (!qw) qw = w.rot;
  if (!kw) kw = w.rot + qn;
  HIP_TRY(hipMemcpyAsync(qw, q, qn * 4, hipMemcpyDeviceToDevice, s), "copy q");
  HIP_TRY(hipMemcpyAsync(kw, k, kn * 4, hipMemcpyDeviceToDevice, s), "copy k");
  st = launch_rope_append_dev(c, qw, kw, v, 1, position, n_heads, n_kv_heads, head_dim, k_cache,
                              v_cache, cap, s);
  if (!st) st = run_generic(c, qw, k_cache, v_cache, kv_stride, out, n_heads, n_kv_heads, head_dim,
                            position, s);
  return st ? st : set_ok();
}

}  // namespace

extern "C" int bnr_dev_decode_step(bnr_ctx *c, const float *q, const float *k, const float *v,
                                   size_t position, size_t n_heads, size_t n_kv_heads,
                                   size_t head_dim, float theta, float *k_cache, float *v_cache,
                                   size_t cap, float *out, float *q_rot, float *k_rot,
                                   void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rope(head_dim, theta);
  if (!st) st = check_rows(position, cap);
  if (st) return st;
  if (!q || !k || !v || !k_cache || !v_cache || !out) return err_backend("decode_step: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  return decode_step_locked(c, q, k, v, position, n_heads, n_kv_heads, head_dim, theta, k_cache,
                            v_cache, cap, out, q_rot, k_rot, (hipStream_t)stream);
}

extern "C" int bnr_dev_decode_step_batched(bnr_ctx *c, const float *q, const float *k,
                                           const float *v, const int32_t *positions, size_t batch,
                                           size_t n_heads, size_t n_kv_heads, size_t head_dim,
                                           float theta, float *k_caches, float *v_caches,
                                           size_t cap, float *out, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rope(head_dim, theta);
  if (st) return st;
  if (batch == 0) return set_ok();
  if (!positions || !q || !k || !v || !k_caches || !v_caches || !out)
    return err_backend("decode_step_batched: NULL pointer");
  size_t maxp = 0;
  for (size_t b = 0; b < batch; ++b) {
    if (positions[b] < 0)
      return err_shape("position >= 0", fmt("positions[%zu] = %d", b, positions[b]));
    maxp = std::max(maxp, (size_t)positions[b]);
  }
  st = check_rows(maxp, cap);
  if (st) return st;
  if (!fast_shape(n_heads, n_kv_heads, head_dim))
    return err_config(fmt("batched decode needs head_dim %d and n_heads/n_kv_heads in {1,2,4}, got "
                          "head_dim %zu, n_heads %zu, n_kv_heads %zu",
                          kHeadDim, head_dim, n_heads, n_kv_heads));
  if (!(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(k_caches) && aligned16(v_caches)))
    return err_shape("16-byte aligned device pointers", "an unaligned pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  st = ensure_table(c, std::max<size_t>((size_t)maxp + 1, cap) - 1, head_dim, theta);
  if (st) return st;
  hipStream_t s = (hipStream_t)stream;
  const long long qs = (long long)(n_heads * head_dim), ks = (long long)(n_kv_heads * head_dim);
  const long long cs = (long long)(n_kv_heads * cap * head_dim);
  for (size_t b0 = 0; b0 < batch; b0 += kMaxBatchPerLaunch) {
    const int nb = (int)std::min<size_t>(kMaxBatchPerLaunch, batch - b0);
    DecodeArgs a{};
    a.q = q + b0 * qs;
    a.k_new = k + b0 * ks;
    a.v_new = v + b0 * ks;
    a.k_cache = k_caches + b0 * cs;
    a.v_cache = v_caches + b0 * cs;
    a.q_bstride = qs;
    a.kn_bstride = ks;
    a.cache_bstride = cs;
    a.out_bstride = qs;
    a.kv_stride = (long long)(cap * head_dim);
    a.out = out + b0 * qs;
    a.cos_tab = c->d_cos;
    a.sin_tab = c->d_sin;
    st = run_decode(c, a, positions + b0, nb, (int)n_kv_heads, (int)(n_heads / n_kv_heads), cap,
                    s);
    if (st) return st;
  }
  return set_ok();
}

namespace {

// Whether prefill attention of this shape runs the tiled kernels.  They take
// at most 65535 query tiles (the grid's y extent) and int positions; longer
// launches run as per-row decodes.
bool prefill_tiled(size_t n_tokens, size_t start_pos, size_t n_heads, size_t n_kv_heads,
                   size_t head_dim, const void *q, const void *k_cache, const void *v_cache,
                   const void *out) {
  return head_dim == (size_t)kHeadDim && prefill_supported((int)(n_heads / n_kv_heads)) &&
         aligned16(q) && aligned16(k_cache) && aligned16(v_cache) && aligned16(out) &&
         n_tokens <= (size_t)kPrefillMaxTokens && start_pos + n_tokens <= (size_t)INT32_MAX;
}

// Stream-K where every query tile has about as many keys as the next (a
// cached prefix at least as long as the new tokens, which are more than 512)
// and no paired launch is planned, or the prefix is at least twice as long:
// 1024 after 3000 303 us against 316 us for a paired launch; 1024 after
// 1024 153 us against 150 us paired (MI355X, graph-timed).  Chunked or paired
// launches otherwise (N = 1024 from an empty cache: 54-62 vs 85 us, 4096:
// 671 vs 710 us).
bool prefill_streamk_shape(const bnr_ctx *c, size_t n_tokens, size_t start_pos) {
  return c->pf_chunk_tiles <= 0 &&
         (c->pf_mode == kPrefillStreamK ||
          (c->pf_mode == kPrefillAuto && start_pos >= n_tokens && n_tokens > 512));
}

// Prefill attention with c->mu held.
int prefill_attention_locked(bnr_ctx *c, const float *q, const float *k_cache,
                             const float *v_cache, size_t cap, float *out, size_t n_tokens,
                             size_t start_pos, size_t n_heads, size_t n_kv_heads, size_t head_dim,
                             hipStream_t s) {
  int st = BNR_OK;
  const long long qs = (long long)(n_heads * head_dim);
  const long long kv_stride = (long long)(cap * head_dim);
  const int group = (int)(n_heads / n_kv_heads);
  if (prefill_tiled(n_tokens, start_pos, n_heads, n_kv_heads, head_dim, q, k_cache, v_cache, out)) {
    PrefillArgs pa{};
    pa.q = q;
    pa.k_cache = k_cache;
    pa.v_cache = v_cache;
    pa.kv_stride = kv_stride;
    pa.out = out;
    pa.n_tokens = (int)n_tokens;
    pa.start_pos = (int)start_pos;
    pa.n_heads = (int)n_heads;
    pa.n_kv = (int)n_kv_heads;
    pa.scale_log2 = 1.4426950408889634f / sqrtf((float)kHeadDim);
    pa.n_qtiles = (int)((n_tokens + 31) / 32);
    pa.timeline = c->timeline;
    const int per_cu = group >= 8 ? 1 : 2;  // resident workgroups per CU (registers, LDS)
    bool streamk = prefill_streamk_shape(c, n_tokens, start_pos);
    if (streamk && c->pf_mode == kPrefillAuto && start_pos < 2 * n_tokens)
      streamk = !plan_prefill_cached(c, (int)n_tokens, (int)start_pos, (int)n_kv_heads, group,
                                     (long long)cap)
                     .choice.pairs;
    int pair_slots = -1;  // a paired launch: its partial-state slots per kv head
    if (!streamk) {
      if (c->pf_chunk_tiles > 0) {
        pa.chunk_tiles = c->pf_chunk_tiles;
        pa.balanced = c->pf_balanced == 1;
        pa.q16 = c->pf_q16 == 1;
      } else {
        const PrefillPlanEntry e = plan_prefill_cached(c, (int)n_tokens, (int)start_pos,
                                                       (int)n_kv_heads, group, (long long)cap);
        pa.chunk_tiles = e.choice.tiles;
        pa.balanced = e.choice.balanced;
        pa.q16 = e.choice.q16;
        if (e.choice.pairs) {
          pa.pair_bins = e.pairs.bins;
          pa.pair_cu = c->n_cu;
          std::memcpy(pa.pair_piece, e.pairs.piece, sizeof(pa.pair_piece));
          pair_slots = e.pairs.n_slots;
        }
      }
    } else {
      pa.chunk_tiles = kPrefillNoSplit;
    }
    PrefillPlan plan = prefill_plan((int)n_tokens, (int)start_pos, pa.chunk_tiles);
    while (plan.n_items > 65535)  // grid y limit
      plan = prefill_plan((int)n_tokens, (int)start_pos, pa.chunk_tiles *= 2);
    pa.n_items = plan.n_items;
    prefill_order(pa);
    {
      // Partial states and tickets, sized -- whatever this launch needs --
      // for every launch on a cache of `cap` rows, so that later calls on it
      // (also under HIP graph capture) never allocate: stream-K launches keep
      // two states per resident workgroup; a planned chunk size keeps to
      // prefill_item_budget (kv head, item) pairs; a forced one (tuning) to
      // T = cap/32 query tiles of at most ceil(T / chunk) chunks each.
      const long long T = ((long long)cap + 31) / 32;
      long long items = c->pf_chunk_tiles > 0
                            ? (long long)n_kv_heads * T * ((T + pa.chunk_tiles - 1) / pa.chunk_tiles)
                            : prefill_item_budget((long long)cap, (int)n_kv_heads);
      if (plan.split) items = std::max<long long>(items, (long long)n_kv_heads * plan.n_items);
      items = std::max<long long>(items, 2LL * c->n_cu * per_cu);
      st = ensure_buf(&c->pf_ws, &c->pf_ws_floats, (size_t)items * group * 66 * 64,
                      "prefill workspace alloc");
      if (st) return st;
      // tickets: one per (kv head, query tile, 16-query half)
      st = ensure_zeroed(&c->pf_counters, &c->n_pf_counters,
                         (size_t)n_kv_heads * std::max<long long>(T, pa.n_qtiles) * 2 *
                             kCounterStride);
      if (st) return st;
    }
    if (streamk) {
      // Equal runs of tile products over the resident workgroups.
      prefill_streamk_units(pa);
      pa.ws = c->pf_ws;
      pa.counters = c->pf_counters;
      const long long slots = c->pf_sk_wgs > 0 ? std::min(c->pf_sk_wgs, c->n_cu * per_cu)
                                                : (long long)c->n_cu * per_cu;
      const int wgs = (int)std::min<long long>(pa.sk_units, slots);
      HIP_TRY(launch_prefill_streamk(pa, group, wgs, s), "prefill launch");
      return set_ok();
    }
    if (plan.split || pair_slots >= 0) {
      pa.ws = c->pf_ws;
      pa.counters = c->pf_counters;
    }
    // slots of the pieces' partial states (within the reservation above:
    // the planner keeps them to prefill_item_budget)
    if (pair_slots >= 0) pa.n_items = std::max(pair_slots, 1);
    int pwgs = 0;
    if (c->pf_mode == kPrefillQueue) pa.q16 = pa.pair_bins = 0;  // the persistent kernel runs whole tiles
    if (c->pf_mode == kPrefillQueue) {
      st = ensure_zeroed(&c->pf_queue, &c->n_pf_queue, 2 * kCounterStride);
      if (st) return st;
      pa.queue = c->pf_queue;
      pwgs = (int)std::min<long long>((long long)n_kv_heads * plan.n_items, (long long)c->n_cu * per_cu);
    }
    HIP_TRY(launch_prefill(pa, group, pwgs, s), "prefill launch");
    return set_ok();
  }
  if (fast_shape(n_heads, n_kv_heads, head_dim) && aligned16(q) && aligned16(k_cache) &&
      aligned16(v_cache)) {
    // Each query row is a decode over the shared cache at its own position.
    int pos[kMaxBatchPerLaunch];
    for (size_t t0 = 0; t0 < n_tokens; t0 += kMaxBatchPerLaunch) {
      const int nb = (int)std::min<size_t>(kMaxBatchPerLaunch, n_tokens - t0);
      for (int i = 0; i < nb; ++i) pos[i] = (int)(start_pos + t0 + i);
      DecodeArgs a{};
      a.q = q + t0 * qs;
      a.k_cache = const_cast<float *>(k_cache);
      a.v_cache = const_cast<float *>(v_cache);
      a.q_bstride = qs;
      a.out_bstride = qs;
      a.kv_stride = kv_stride;
      a.out = out + t0 * qs;
      st = run_decode(c, a, pos, nb, (int)n_kv_heads, (int)(n_heads / n_kv_heads), cap, s);
      if (st) return st;
    }
    return set_ok();
  }
  for (size_t i = 0; i < n_tokens; ++i) {
    st = run_generic(c, q + i * qs, k_cache, v_cache, kv_stride, out + i * qs, n_heads, n_kv_heads,
                     head_dim, start_pos + i, s);
    if (st) return st;
  }
  return set_ok();
}

}  // namespace

extern "C" int bnr_dev_prefill_attention(bnr_ctx *c, const float *q, const float *k_cache,
                                         const float *v_cache, size_t cap, float *out,
                                         size_t n_tokens, size_t start_pos, size_t n_heads,
                                         size_t n_kv_heads, size_t head_dim, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (st) return st;
  if (n_tokens == 0) return set_ok();
  st = check_rows(start_pos + n_tokens - 1, cap);
  if (st) return st;
  if (!q || !k_cache || !v_cache || !out) return err_backend("prefill_attention: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  st = prefill_attention_locked(c, q, k_cache, v_cache, cap, out, n_tokens, start_pos, n_heads,
                                n_kv_heads, head_dim, (hipStream_t)stream);
  return st ? st : set_ok();
}

// bnr_dev_rope_append then bnr_dev_prefill_attention under one lock: the
// first's checks, then the output pointer's.
extern "C" int bnr_dev_prefill(bnr_ctx *c, float *q, float *k, const float *v, size_t n_tokens,
                               size_t start_pos, size_t n_heads, size_t n_kv_heads,
                               size_t head_dim, float theta, float *k_cache, float *v_cache,
                               size_t cap, float *out, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_heads(n_heads, n_kv_heads, head_dim);
  if (!st) st = check_rope(head_dim, theta);
  if (st) return st;
  if (n_tokens == 0) return set_ok();
  st = check_rows(start_pos + n_tokens - 1, cap);
  if (st) return st;
  if (!q || !k || !v || !k_cache || !v_cache) return err_backend("rope_append: NULL pointer");
  if (!out) return err_backend("prefill_attention: NULL pointer");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  hipStream_t s = (hipStream_t)stream;
  st = ensure_table(c, std::max(start_pos + n_tokens, cap) - 1, head_dim, theta);
  if (st) return st;
  st = launch_rope_append_dev(c, q, k, v, n_tokens, start_pos, n_heads, n_kv_heads, head_dim,
                              k_cache, v_cache, cap, s);
  if (st) return st;
  st = prefill_attention_locked(c, q, k_cache, v_cache, cap, out, n_tokens, start_pos, n_heads,
                                n_kv_heads, head_dim, s);
  return st ? st : set_ok();
}

// ---------------------------------------------------------------------------
// LM head with i8 weights
// ---------------------------------------------------------------------------
namespace {

int check_lm_head(size_t hidden_len, size_t weights_len, size_t scales_len, size_t out_len,
                  size_t vocab_size, size_t hidden_size) {
  if (hidden_len != SIZE_MAX && hidden_len != hidden_size)
    return err_shape(fmt("hidden.len() == %zu", hidden_size), fmt("hidden.len() == %zu", hidden_len));
  if (hidden_size != 0 && vocab_size > SIZE_MAX / hidden_size)
    return err_shape("weight size fits usize", "overflow");
  if (weights_len != SIZE_MAX && weights_len != vocab_size * hidden_size)
    return err_shape(fmt("weights_i8.len() == %zu * %zu", vocab_size, hidden_size),
                     fmt("weights_i8.len() == %zu", weights_len));
  if (scales_len != SIZE_MAX && scales_len != vocab_size)
    return err_shape(fmt("scales.len() == %zu", vocab_size), fmt("scales.len() == %zu", scales_len));
  if (out_len != SIZE_MAX && out_len != vocab_size)
    return err_shape(fmt("output.len() == %zu", vocab_size), fmt("output.len() == %zu", out_len));
  if (hidden_size > (size_t)INT32_MAX)
    return err_backend("lm_head_matmul_i8: hidden_size beyond 2^31 is not supported");
  return BNR_OK;
}

int run_lm_head(const float *hidden, const int8_t *w, const float *scales, float *out,
                size_t vocab_size, size_t hidden_size, hipStream_t s) {
  LmHeadArgs a{};
  a.hidden = hidden;
  a.weight = w;
  a.scales = scales;
  a.out = out;
  a.vocab_size = (long long)vocab_size;
  a.hidden_size = (int)hidden_size;
  const bool vec = hidden_size % 16 == 0 && ((uintptr_t)w % 16) == 0 && ((uintptr_t)hidden % 16) == 0;
  HIP_TRY(launch_lm_head_i8(a, vec, s), "lm_head launch");
  return BNR_OK;
}

}  // namespace

extern "C" int bnr_lm_head_matmul_i8_into(bnr_ctx *c, const float *hidden, size_t hidden_len,
                                          const int8_t *weights_i8, size_t weights_len,
                                          const float *scales, size_t scales_len, float *output,
                                          size_t out_len, size_t vocab_size, size_t hidden_size) {
  if (!c) return err_backend("context is NULL");
  int st = check_lm_head(hidden_len, weights_len, scales_len, out_len, vocab_size, hidden_size);
  if (st) return st;
  if (vocab_size == 0) return set_ok();
  if ((hidden_size && (!hidden || !weights_i8)) || !scales || !output)
    return err_backend("lm_head_matmul_i8_into: NULL slice");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  const uint8_t *dw = nullptr, *dsc = nullptr;
  if (weights_len) {
    st = mirror_bytes(c, weights_i8, weights_len, &dw);
    if (st) return st;
  }
  st = mirror_bytes(c, scales, scales_len * sizeof(float), &dsc);
  if (st) return st;
  st = ensure_buf(&c->d_q, &c->d_q_n, std::max<size_t>(hidden_size, 4), "staging alloc");
  if (st) return st;
  st = ensure_buf(&c->d_out, &c->d_out_n, vocab_size, "staging alloc");
  if (st) return st;
  if (hidden_size) {
    st = put_host(c, c->d_q, {{hidden, hidden_size * 4}}, "upload hidden");
    if (st) return st;
  }
  st = run_lm_head(c->d_q, (const int8_t *)dw, (const float *)dsc, c->d_out, vocab_size,
                   hidden_size, c->stream);
  if (st) return st;
  st = get_host(c, output, c->d_out, vocab_size * 4, "lm_head_matmul_i8_into");
  return st ? st : set_ok();
}

extern "C" int bnr_dev_lm_head_matmul_i8(bnr_ctx *c, const float *hidden, const int8_t *weights_i8,
                                         const float *scales, float *output, size_t vocab_size,
                                         size_t hidden_size, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_lm_head(SIZE_MAX, SIZE_MAX, SIZE_MAX, SIZE_MAX, vocab_size, hidden_size);
  if (st) return st;
  if (vocab_size == 0) return set_ok();
  if ((hidden_size && (!hidden || !weights_i8)) || !scales || !output)
    return err_backend("lm_head_matmul_i8: NULL pointer");
  DeviceGuard dg(c->device);
  st = run_lm_head(hidden, weights_i8, scales, output, vocab_size, hidden_size, (hipStream_t)stream);
  if (st) return st;
  return set_ok();
}

extern "C" int bnr_dev_ternary_gemv_preq(bnr_ctx *c, const uint8_t *weight_packed,
                                         float weight_scale, const int8_t *activation_q,
                                         float act_absmax, float *output, size_t out_features,
                                         size_t in_features, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_gemv(SIZE_MAX, weight_scale, SIZE_MAX, act_absmax, SIZE_MAX, out_features,
                      in_features);
  if (st) return st;
  if (out_features == 0) return set_ok();
  if ((in_features && (!weight_packed || !activation_q)) || !output)
    return err_backend("ternary_gemv_preq: NULL pointer");
  DeviceGuard dg(c->device);
  st = run_gemv(weight_packed, weight_scale, activation_q, act_absmax, output, out_features,
                in_features, (hipStream_t)stream);
  if (st) return st;
  return set_ok();
}

namespace {

// Grouped GEMV launch; act_absmax_dev non-null: the activation scale is read
// from device memory (produced by the fused norm/quantise kernel).
int run_gemv_group(bnr_ctx *c, size_t n, const uint8_t *const *weight_packed,
                   const float *weight_scales, const int8_t *activation_q, float act_absmax,
                   const float *act_absmax_dev, float *const *outputs,
                   const size_t *out_features, size_t in_features, hipStream_t stream) {
  if (!c) return err_backend("context is NULL");
  if (n == 0 || n > (size_t)kMaxGemvGroup)
    return err_config(fmt("ternary GEMV group size must be 1..%d, got %zu", kMaxGemvGroup, n));
  if (!weight_packed || !weight_scales || !outputs || !out_features)
    return err_backend("ternary_gemv_preq_group: NULL array");
  TernaryGemvGroupArgs g{};
  g.n = (int)n;
  g.act = activation_q;
  g.in_features = (int)in_features;
  g.packed_cols = (long long)((in_features + 3) / 4);
  g.act_absmax_dev = act_absmax_dev;
  bool vec = g.packed_cols % 16 == 0 && ((uintptr_t)activation_q % 16) == 0;
  int wgs = 0;
  for (size_t i = 0; i < n; ++i) {
    int st = check_gemv(SIZE_MAX, weight_scales[i], SIZE_MAX, act_absmax_dev ? 1.0f : act_absmax,
                        SIZE_MAX, out_features[i], in_features);
    if (st) return st;
    if (out_features[i] && ((in_features && (!weight_packed[i] || !activation_q)) || !outputs[i]))
      return err_backend("ternary_gemv_preq_group: NULL pointer");
    g.weight[i] = weight_packed[i];
    g.out[i] = outputs[i];
    g.weight_scale[i] = weight_scales[i];
    volatile float ws_as = weight_scales[i] * act_absmax;
    g.scale[i] = ws_as / 127.0f;
    g.out_features[i] = (int)out_features[i];
    g.wg_off[i] = wgs;
    wgs += (int)((out_features[i] + 15) / 16);
    vec = vec && ((uintptr_t)weight_packed[i] % 16) == 0;
  }
  for (size_t i = n; i <= (size_t)kMaxGemvGroup; ++i) g.wg_off[i] = wgs;
  if (wgs == 0) return set_ok();
  DeviceGuard dg(c->device);
  HIP_TRY(launch_ternary_gemv_group(g, vec, stream), "ternary_gemv group launch");
  return set_ok();
}

}  // namespace

extern "C" int bnr_dev_ternary_gemv_preq_group(bnr_ctx *c, size_t n,
                                               const uint8_t *const *weight_packed,
                                               const float *weight_scales,
                                               const int8_t *activation_q, float act_absmax,
                                               float *const *outputs, const size_t *out_features,
                                               size_t in_features, void *stream) {
  return run_gemv_group(c, n, weight_packed, weight_scales, activation_q, act_absmax, nullptr,
                        outputs, out_features, in_features, (hipStream_t)stream);
}

extern "C" int bnr_dev_ternary_gemv_preq_group_devscale(
    bnr_ctx *c, size_t n, const uint8_t *const *weight_packed, const float *weight_scales,
    const int8_t *activation_q, const float *act_absmax, float *const *outputs,
    const size_t *out_features, size_t in_features, void *stream) {
  if (!act_absmax) return err_backend("ternary_gemv_preq_group_devscale: NULL act_absmax");
  return run_gemv_group(c, n, weight_packed, weight_scales, activation_q, 1.0f, act_absmax,
                        outputs, out_features, in_features, (hipStream_t)stream);
}

extern "C" int bnr_dev_ternary_gemv_norm_group(
    bnr_ctx *c, size_t n, const uint8_t *const *weight_packed, const float *weight_scales,
    int mode, const float *a, const float *b, const float *gamma, float eps, float *h_out,
    float *const *outputs, const size_t *out_features, size_t in_features, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (n == 0 || n > (size_t)kMaxGemvGroup)
    return err_config(fmt("ternary GEMV group size must be 1..%d, got %zu", kMaxGemvGroup, n));
  if (mode != BNR_GLUE_PLAIN && mode != BNR_GLUE_RESIDUAL && mode != BNR_GLUE_SQRELU)
    return err_config(fmt("unknown norm_quant mode %d", mode));
  if (eps <= 0.0f || !std::isfinite(eps))
    return err_quant("eps must be finite and > 0, got " + rust_f32(eps));
  if (in_features == 0) return err_quant("cannot quantise an empty activation vector");
  if (in_features > (size_t)kMaxNormGemvK)
    return err_backend(fmt("ternary_gemv_norm_group: in_features %zu > %d is not supported "
                           "(use bnr_dev_norm_quant + bnr_dev_ternary_gemv_preq_group_devscale)",
                           in_features, kMaxNormGemvK));
  if (!weight_packed || !weight_scales || !outputs || !out_features || !a || !gamma ||
      (mode != BNR_GLUE_PLAIN && !b) || (mode == BNR_GLUE_RESIDUAL && !h_out))
    return err_backend("ternary_gemv_norm_group: NULL pointer");
  if (h_out && (h_out == a || h_out == b))
    return err_backend("ternary_gemv_norm_group: h_out must not alias a or b");
  TernaryGemvGroupArgs g{};
  g.n = (int)n;
  g.in_features = (int)in_features;
  g.packed_cols = (long long)((in_features + 3) / 4);
  bool vec = g.packed_cols % 16 == 0;
  // Rows per workgroup: each workgroup reads all of a (and b) and gamma, so
  // the launch takes the most rows per workgroup that still leave it
  // gemv_norm_min_wgs workgroups.
  int rows = 16;
  for (int r : {64, 32}) {
    long long w = 0;
    for (size_t i = 0; i < n; ++i) w += ((long long)out_features[i] + r - 1) / r;
    if (w >= c->gemv_norm_min_wgs) {
      rows = r;
      break;
    }
  }
  int wgs = 0;
  for (size_t i = 0; i < n; ++i) {
    int st = check_gemv(SIZE_MAX, weight_scales[i], SIZE_MAX, 1.0f, SIZE_MAX, out_features[i],
                        in_features);
    if (st) return st;
    if (out_features[i] && (!weight_packed[i] || !outputs[i]))
      return err_backend("ternary_gemv_norm_group: NULL pointer");
    g.weight[i] = weight_packed[i];
    g.out[i] = outputs[i];
    g.weight_scale[i] = weight_scales[i];
    g.out_features[i] = (int)out_features[i];
    g.wg_off[i] = wgs;
    wgs += (int)((out_features[i] + rows - 1) / rows);
    vec = vec && ((uintptr_t)weight_packed[i] % 16) == 0;
  }
  for (size_t i = n; i <= (size_t)kMaxGemvGroup; ++i) g.wg_off[i] = wgs;
  if (wgs == 0) return set_ok();
  GemvNormArgs p{};
  p.mode = mode;
  p.a = a;
  p.b = b;
  p.gamma = gamma;
  p.eps = eps;
  p.h_out = mode == BNR_GLUE_RESIDUAL ? h_out : nullptr;
  p.rows = rows;
  // The vector path also reads the activation vectors as float4 groups.
  vec = vec && in_features % 16 == 0 && aligned16(a) && aligned16(gamma) &&
        (mode == BNR_GLUE_PLAIN || aligned16(b)) && (!p.h_out || aligned16(p.h_out));
  DeviceGuard dg(c->device);
  HIP_TRY(launch_ternary_gemv_norm(g, p, vec, (hipStream_t)stream), "ternary_gemv_norm launch");
  return set_ok();
}

// ---------------------------------------------------------------------------
// Layer glue
// ---------------------------------------------------------------------------
namespace {

// norm::rms_norm checks (bitnet-cpu/src/norm.rs:77-97), in its order.
int check_rms_norm(size_t in_len, size_t w_len, float eps, size_t out_len) {
  if (in_len != w_len)
    return err_shape(fmt("input.len() == weight.len() = %zu", w_len), fmt("input.len() = %zu", in_len));
  if (in_len != out_len)
    return err_shape(fmt("input.len() == output.len() = %zu", in_len), fmt("output.len() = %zu", out_len));
  if (eps <= 0.0f || !std::isfinite(eps))
    return err_quant("eps must be finite and > 0, got " + rust_f32(eps));
  if (in_len > (size_t)INT32_MAX) return err_backend("rms_norm: length beyond 2^31 is not supported");
  return BNR_OK;
}

int run_norm_quant(bnr_ctx *c, int mode, const float *a, const float *b, const float *gamma,
                   float eps, size_t n, float *h_out, float *y_out, int8_t *q_out,
                   float *scale_out, float *act_absmax, hipStream_t s, unsigned *done = nullptr,
                   unsigned seq = 0) {
  NormQuantArgs na{};
  na.done = done;
  na.seq = seq;
  na.mode = mode;
  na.a = a;
  na.b = b;
  na.gamma = gamma;
  na.eps = eps;
  na.n = (int)n;
  na.h_out = h_out;
  na.y_out = y_out;
  na.q_out = q_out;
  na.scale_out = scale_out;
  na.act_absmax = act_absmax;
  DeviceGuard dg(c->device);
  HIP_TRY(launch_norm_quant(na, s), "norm_quant launch");
  return BNR_OK;
}

}  // namespace

extern "C" int bnr_rms_norm(bnr_ctx *c, const float *input, size_t in_len, const float *weight,
                            size_t w_len, float eps, float *output, size_t out_len) {
  if (!c) return err_backend("context is NULL");
  int st = check_rms_norm(in_len, w_len, eps, out_len);
  if (st) return st;
  if (in_len == 0) return set_ok();
  if (!input || !weight || !output) return err_backend("rms_norm: NULL slice");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  const uint8_t *dw = nullptr;
  st = mirror_bytes(c, weight, w_len * sizeof(float), &dw);
  if (st) return st;
  // input and output in the zero-copy staging: [input | output]
  const size_t is = round4(in_len);
  st = ensure_zc(c, is + in_len);
  if (st) return st;
  std::memcpy(c->h_zc, input, in_len * sizeof(float));
  const bool sig = ensure_sig(c);
  const unsigned seq = sig ? next_seq(c) : 0;
  st = run_norm_quant(c, kGluePlain, c->d_zc, nullptr, (const float *)dw, eps, in_len, nullptr,
                      c->d_zc + is, nullptr, nullptr, nullptr, c->stream, sig ? c->d_sig : nullptr,
                      seq);
  if (st) return st;
  st = sig ? host_wait_words(c, 1, seq, "rms_norm") : host_wait(c, "rms_norm");
  if (st) return st;
  std::memcpy(output, c->h_zc + is, in_len * sizeof(float));
  return set_ok();
}

extern "C" int bnr_sqrelu_gate(bnr_ctx *c, const float *gate, size_t g_len, const float *up,
                               size_t u_len, float *out, size_t out_len) {
  if (!c) return err_backend("context is NULL");
  if (g_len != u_len || g_len != out_len)
    return err_shape(fmt("gate.len() == up.len() == out.len() = %zu", g_len),
                     fmt("up.len()=%zu, out.len()=%zu", u_len, out_len));
  if (g_len == 0) return set_ok();
  if (!gate || !up || !out) return err_backend("sqrelu_gate: NULL slice");
  std::lock_guard<std::mutex> lk(c->mu);
  DeviceGuard dg(c->device);
  // gate, up and the output in the zero-copy staging: [gate | up | out]
  const size_t gs = round4(g_len);
  int st = ensure_zc(c, 3 * gs);
  if (st) return st;
  float *h = c->h_zc, *d = c->d_zc;
  std::memcpy(h, gate, g_len * sizeof(float));
  std::memcpy(h + gs, up, g_len * sizeof(float));
  const long long words = sqrelu_blocks((long long)g_len);
  const bool sig = words <= kSignalWords && ensure_sig(c);
  const unsigned seq = sig ? next_seq(c) : 0;
  HIP_TRY(launch_sqrelu(d, d + gs, d + 2 * gs, (long long)g_len, c->stream,
                        sig ? c->d_sig : nullptr, seq),
          "sqrelu launch");
  st = sig ? host_wait_words(c, (int)words, seq, "sqrelu_gate") : host_wait(c, "sqrelu_gate");
  if (st) return st;
  std::memcpy(out, h + 2 * gs, g_len * sizeof(float));
  return set_ok();
}

extern "C" int bnr_dev_rms_norm(bnr_ctx *c, const float *input, const float *weight, float eps,
                                float *output, size_t n, void *stream) {
  if (!c) return err_backend("context is NULL");
  int st = check_rms_norm(n, n, eps, n);
  if (st) return st;
  if (n == 0) return set_ok();
  if (!input || !weight || !output) return err_backend("rms_norm: NULL pointer");
  st = run_norm_quant(c, kGluePlain, input, nullptr, weight, eps, n, nullptr, output, nullptr,
                      nullptr, nullptr, (hipStream_t)stream);
  return st ? st : set_ok();
}

extern "C" int bnr_dev_sqrelu_gate(bnr_ctx *c, const float *gate, const float *up, float *out,
                                   size_t n, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (n == 0) return set_ok();
  if (!gate || !up || !out) return err_backend("sqrelu_gate: NULL pointer");
  DeviceGuard dg(c->device);
  HIP_TRY(launch_sqrelu(gate, up, out, (long long)n, (hipStream_t)stream), "sqrelu launch");
  return set_ok();
}

extern "C" int bnr_dev_residual_add(bnr_ctx *c, float *h, const float *delta, size_t n,
                                    void *stream) {
  if (!c) return err_backend("context is NULL");
  if (n == 0) return set_ok();
  if (!h || !delta) return err_backend("residual_add: NULL pointer");
  DeviceGuard dg(c->device);
  HIP_TRY(launch_residual(h, delta, (long long)n, (hipStream_t)stream), "residual launch");
  return set_ok();
}

extern "C" int bnr_dev_absmax_quantize(bnr_ctx *c, const float *x, int8_t *q_out, float *scale_out,
                                       size_t n, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (n == 0) return err_quant("cannot quantise an empty activation vector");
  if (n > (size_t)INT32_MAX) return err_backend("absmax_quantize: length beyond 2^31 is not supported");
  if (!x || !q_out || !scale_out) return err_backend("absmax_quantize: NULL pointer");
  int st = run_norm_quant(c, kGluePlain, x, nullptr, nullptr, 1.0f, n, nullptr, nullptr, q_out,
                          scale_out, nullptr, (hipStream_t)stream);
  return st ? st : set_ok();
}

extern "C" int bnr_dev_norm_quant(bnr_ctx *c, int mode, const float *a, const float *b,
                                  const float *gamma, float eps, size_t n, float *h_out,
                                  int8_t *q_out, float *act_absmax, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (mode != BNR_GLUE_PLAIN && mode != BNR_GLUE_RESIDUAL && mode != BNR_GLUE_SQRELU)
    return err_config(fmt("unknown norm_quant mode %d", mode));
  int st = check_rms_norm(n, n, eps, n);
  if (st) return st;
  if (n == 0) return err_quant("cannot quantise an empty activation vector");
  if (!a || !gamma || !q_out || !act_absmax || (mode != BNR_GLUE_PLAIN && !b) ||
      (mode == BNR_GLUE_RESIDUAL && !h_out))
    return err_backend("norm_quant: NULL pointer");
  st = run_norm_quant(c, mode, a, b, gamma, eps, n, mode == BNR_GLUE_RESIDUAL ? h_out : nullptr,
                      nullptr, q_out, nullptr, act_absmax, (hipStream_t)stream);
  return st ? st : set_ok();
}

extern "C" int bnr_dev_synchronize(bnr_ctx *c, void *stream) {
  if (!c) return err_backend("context is NULL");
  DeviceGuard dg(c->device);
  HIP_TRY(hipStreamSynchronize((hipStream_t)stream), "synchronize");
  return set_ok();
}

// ---------------------------------------------------------------------------
// Backend-owned KV cache: KVCache (bitnet-model/src/lib.rs:118-315) with its
// buffers in HBM.  One allocation holds, per layer, K then V, each
// head-major [n_kv_heads x max_seq x head_dim].  The bookkeeping
// (layer_lengths, filled_positions) and store_kv's position rules are the
// reference's; the row itself is written by the decode / prefill kernels.
// ---------------------------------------------------------------------------
struct bnr_kv_cache {
  int device = 0;
  size_t n_layers = 0, n_kv = 0, head_dim = 0, max_seq = 0;
  size_t layer_floats = 0;  // n_kv * max_seq * head_dim (one of K or V)
  float *base = nullptr;
  std::vector<size_t> layer_len;
  size_t filled = 0;
  mutable std::mutex mu;  // bookkeeping; calls on one cache are serialised

  float *k(size_t layer) const { return base + 2 * layer * layer_floats; }
  float *v(size_t layer) const { return base + (2 * layer + 1) * layer_floats; }
};

namespace {

int kv_check_layer(const bnr_kv_cache *kc, size_t layer) {
  if (layer >= kc->n_layers)
    return err_shape(fmt("layer < num_hidden_layers (%zu)", kc->n_layers), fmt("layer = %zu", layer));
  return BNR_OK;
}

// store_kv's position rules (lib.rs:204-216) for rows position..position+n-1
// written in order: each row either overwrites a stored one or extends the
// layer by one.
int kv_check_store(const bnr_kv_cache *kc, size_t layer, size_t position, size_t n) {
  int st = kv_check_layer(kc, layer);
  if (st) return st;
  const size_t last = position + n - 1;
  if (last >= kc->max_seq)
    return err_shape(fmt("position < max_seq (%zu)", kc->max_seq), fmt("position = %zu", last));
  if (position > kc->layer_len[layer])
    return err_shape(fmt("position <= layer_len_positions (%zu)", kc->layer_len[layer]),
                     fmt("position = %zu", position));
  return BNR_OK;
}

void kv_mark_stored(bnr_kv_cache *kc, size_t layer, size_t position, size_t n) {
  kc->layer_len[layer] = std::max(kc->layer_len[layer], position + n);
}

}  // namespace

extern "C" int bnr_kv_cache_create(bnr_ctx *c, size_t n_layers, size_t n_kv_heads, size_t head_dim,
                                   size_t max_seq, bnr_kv_cache **out) {
  if (!out) return err_backend("kv_cache_create: NULL out");
  *out = nullptr;
  if (!c) return err_backend("context is NULL");
  if (n_layers == 0) return err_config("num_hidden_layers must be > 0");
  if (n_kv_heads == 0) return err_config("n_kv_heads must be > 0");
  if (head_dim == 0) return err_shape("head_dim > 0", "head_dim = 0");
  if (max_seq == 0) return err_shape("max_seq > 0", "max_seq = 0");
  const size_t per = n_kv_heads * max_seq * head_dim;
  if (per / n_kv_heads / head_dim != max_seq || per > SIZE_MAX / 8 / n_layers)
    return err_shape("a cache size that fits in memory", "an overflowing size");
  const size_t bytes = 2 * n_layers * per * sizeof(float);
  DeviceGuard dg(c->device);
  auto *kc = new (std::nothrow) bnr_kv_cache();
  if (!kc) return err_backend("kv cache: out of host memory");
  kc->device = c->device;
  kc->n_layers = n_layers;
  kc->n_kv = n_kv_heads;
  kc->head_dim = head_dim;
  kc->max_seq = max_seq;
  kc->layer_floats = per;
  kc->layer_len.assign(n_layers, 0);
  hipError_t e = hipMalloc((void **)&kc->base, bytes);
  if (e == hipSuccess) e = hipMemset(kc->base, 0, bytes);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    if (kc->base) (void)hipFree(kc->base);
    delete kc;
    return err_hip(e, "kv cache alloc");
  }
  *out = kc;
  return set_ok();
}

extern "C" void bnr_kv_cache_destroy(bnr_kv_cache *kc) {
  if (!kc) return;
  DeviceGuard dg(kc->device);
  (void)hipDeviceSynchronize();  // kernels in flight may still use the cache
  (void)hipFree(kc->base);
  delete kc;
}

extern "C" int bnr_kv_cache_clear(bnr_kv_cache *kc) {
  if (!kc) return err_backend("kv cache is NULL");
  std::lock_guard<std::mutex> lk(kc->mu);
  DeviceGuard dg(kc->device);
  HIP_TRY(hipDeviceSynchronize(), "kv cache clear");
  HIP_TRY(hipMemset(kc->base, 0, 2 * kc->n_layers * kc->layer_floats * sizeof(float)),
          "kv cache clear");
  HIP_TRY(hipDeviceSynchronize(), "kv cache clear");
  std::fill(kc->layer_len.begin(), kc->layer_len.end(), (size_t)0);
  kc->filled = 0;
  return set_ok();
}

extern "C" int bnr_kv_cache_advance(bnr_kv_cache *kc, size_t n) {
  if (!kc) return err_backend("kv cache is NULL");
  std::lock_guard<std::mutex> lk(kc->mu);
  // KVCache::advance asserts filled_positions < max_seq before each step
  // (and panics); here nothing advances and the message is an error.
  if (n > kc->max_seq - kc->filled)
    return err_backend(fmt("KVCache::advance overflow: filled_positions=%zu max_seq=%zu",
                           kc->filled, kc->max_seq));
  kc->filled += n;
  return set_ok();
}

extern "C" size_t bnr_kv_cache_len(const bnr_kv_cache *kc) {
  if (!kc) return 0;
  std::lock_guard<std::mutex> lk(kc->mu);
  return kc->filled;
}

extern "C" int bnr_kv_cache_layer_len(bnr_kv_cache *kc, size_t layer, size_t *len) {
  if (!kc || !len) return err_backend("kv_cache_layer_len: NULL pointer");
  std::lock_guard<std::mutex> lk(kc->mu);
  int st = kv_check_layer(kc, layer);
  if (st) return st;
  *len = kc->layer_len[layer];
  return set_ok();
}

extern "C" int bnr_kv_cache_layer(bnr_kv_cache *kc, size_t layer, float **k, float **v) {
  if (!kc || !k || !v) return err_backend("kv_cache_layer: NULL pointer");
  int st = kv_check_layer(kc, layer);
  if (st) return st;
  *k = kc->k(layer);
  *v = kc->v(layer);
  return set_ok();
}

extern "C" int bnr_kv_decode(bnr_ctx *c, bnr_kv_cache *kc, size_t layer, float *q, size_t q_len,
                             float *k, size_t k_len, const float *v, size_t v_len,
                             size_t position, size_t n_heads, float theta, float *output,
                             size_t out_len) {
  if (!c) return err_backend("context is NULL");
  if (!kc) return err_backend("kv cache is NULL");
  const size_t hd = kc->head_dim, nkv = kc->n_kv, kvn = nkv * hd;
  // rope_embed first (RopeCache::new, then apply_rope_cached's lengths:
  // bitnet-cpu/src/rope.rs:101-110, 324-337) ...
  int st = check_rope(hd, theta);
  if (st) return st;
  if (q_len != n_heads * hd)
    return err_shape(fmt("q.len() == %zu * %zu = %zu", n_heads, hd, n_heads * hd),
                     fmt("q.len() = %zu", q_len));
  if (k_len != kvn)
    return err_shape(fmt("k.len() == %zu * %zu = %zu", nkv, hd, kvn), fmt("k.len() = %zu", k_len));
  // ... then store_kv (bitnet-model/src/lib.rs:190-216) ...
  if (v_len != kvn) return err_shape(fmt("v_vec.len() = %zu", kvn), fmt("%zu", v_len));
  std::lock_guard<std::mutex> lk(kc->mu);
  st = kv_check_store(kc, layer, position, 1);
  if (st) return st;
  // ... then masked_attention (bitnet-cpu/src/attention.rs:109-161).
  st = check_heads(n_heads, nkv, hd);
  if (st) return st;
  if (out_len != n_heads * hd)
    return err_shape(fmt("output.len() == n_heads * head_dim = %zu", n_heads * hd),
                     fmt("output.len() = %zu", out_len));
  if (!q || !k || !v || !output) return err_backend("kv_decode: NULL slice");
  if (kc->device != c->device) return err_backend("kv cache and context are on different devices");
  std::lock_guard<std::mutex> lc(c->mu);
  DeviceGuard dg(c->device);
  // Zero-copy staging, [q | k | v | out | rotated q | rotated k], every part
  // 16-byte aligned: the decode kernel reads its inputs from pinned host
  // memory and writes its outputs there, and the call waits for its
  // completion words (a stream synchronisation where the kernel stores none).
  const size_t qs = round4(q_len), ks = round4(kvn), os = round4(out_len);
  const size_t in_n = qs + 2 * ks, back_n = os + qs + ks;
  st = ensure_zc(c, in_n + back_n);
  if (st) return st;
  float *h = c->h_zc;
  std::memcpy(h, q, q_len * sizeof(float));
  std::memcpy(h + qs, k, kvn * sizeof(float));
  std::memcpy(h + qs + ks, v, kvn * sizeof(float));
  float *dq = c->d_zc, *dk = dq + qs, *dv = dk + ks, *dout = dq + in_n, *dqr = dout + os,
        *dkr = dqr + qs;
  const bool sig = (int)nkv <= kSignalWords && ensure_sig(c);
  const unsigned seq = sig ? next_seq(c) : 0;
  bool signals = false;
  st = decode_step_locked(c, dq, dk, dv, position, n_heads, nkv, hd, theta, kc->k(layer),
                          kc->v(layer), kc->max_seq, dout, dqr, dkr, c->stream,
                          sig ? c->d_sig : nullptr, seq, &signals);
  if (st) return st;
  st = signals ? host_wait_words(c, (int)nkv, seq, "kv_decode") : host_wait(c, "kv_decode");
  if (st) return st;
  const float *hb = h + in_n;
  std::memcpy(output, hb, out_len * sizeof(float));
  std::memcpy(q, hb + os, q_len * sizeof(float));
  std::memcpy(k, hb + os + qs, kvn * sizeof(float));
  kv_mark_stored(kc, layer, position, 1);
  return set_ok();
}

extern "C" int bnr_kv_dev_decode(bnr_ctx *c, bnr_kv_cache *kc, size_t layer, const float *q,
                                 const float *k, const float *v, size_t position, size_t n_heads,
                                 float theta, float *out, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (!kc) return err_backend("kv cache is NULL");
  const size_t hd = kc->head_dim, nkv = kc->n_kv;
  int st = check_rope(hd, theta);
  if (st) return st;
  std::lock_guard<std::mutex> lk(kc->mu);
  st = kv_check_store(kc, layer, position, 1);
  if (!st) st = check_heads(n_heads, nkv, hd);
  if (st) return st;
  if (!q || !k || !v || !out) return err_backend("kv_dev_decode: NULL pointer");
  if (kc->device != c->device) return err_backend("kv cache and context are on different devices");
  {
    std::lock_guard<std::mutex> lc(c->mu);
    st = decode_step_locked(c, q, k, v, position, n_heads, nkv, hd, theta, kc->k(layer),
                            kc->v(layer), kc->max_seq, out, nullptr, nullptr, (hipStream_t)stream);
  }
  if (st) return st;
  kv_mark_stored(kc, layer, position, 1);
  return set_ok();
}

extern "C" int bnr_kv_dev_prefill(bnr_ctx *c, bnr_kv_cache *kc, size_t layer, float *q, float *k,
                                  const float *v, size_t n_tokens, size_t start_pos,
                                  size_t n_heads, float theta, float *out, void *stream) {
  if (!c) return err_backend("context is NULL");
  if (!kc) return err_backend("kv cache is NULL");
  int st = check_rope(kc->head_dim, theta);
  if (st) return st;
  std::lock_guard<std::mutex> lk(kc->mu);
  if (n_tokens == 0) {
    st = kv_check_layer(kc, layer);
    return st ? st : set_ok();
  }
  st = kv_check_store(kc, layer, start_pos, n_tokens);
  if (st) return st;
  if (kc->device != c->device) return err_backend("kv cache and context are on different devices");
  st = bnr_dev_prefill(c, q, k, v, n_tokens, start_pos, n_heads, kc->n_kv, kc->head_dim, theta,
                       kc->k(layer), kc->v(layer), kc->max_seq, out, stream);
  if (st) return st;
  kv_mark_stored(kc, layer, start_pos, n_tokens);
  return set_ok();
}
