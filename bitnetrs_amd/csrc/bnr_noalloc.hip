// bnr_noalloc.hip -- the device scratch of bnr_dev_decode_attention_noalloc:
// a file-scope device array that holds the split-K merge state of one decode
// launch (reference-merge accumulators, tickets, exact-path partial states),
// so that the entry point never allocates.  Each GPU holds its own copy of
// the array until the process ends; its address on a device comes from
// hipGetSymbolAddress, taken once per device with that device current.
#include "bnr_internal.h"

#include <hip/hip_runtime.h>

#include <mutex>

namespace bnr {
namespace {

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// Zero the merge state (accumulators and tickets): the kernels leave it zero
// after every launch, so this runs once per device.
__global__ __launch_bounds__(256) void zero_words_kernel(unsigned *p, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};
// The (context, stream) pair whose launches use a device's scratch: every
// launch on one GPU shares the array, so launches from another context or
// stream could overlap with them on the GPU and race on the accumulators
// and tickets.
struct Owner {
  const void *ctx = nullptr;
  const void *stream = nullptr;
};
Owner g_owner[kMaxDevices];

}  // namespace

bool noalloc_claim(int device, const void *ctx, const void *stream) {
  if (device < 0 || device >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lk(g_mu);
  Owner &o = g_owner[device];
  if (!o.ctx) {
    o.ctx = ctx;
    o.stream = stream;
    return true;
  }
  return o.ctx == ctx && o.stream == stream;
}

void noalloc_release(int device, const void *ctx) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_owner[device].ctx == ctx) g_owner[device] = Owner{};
}

hipError_t noalloc_scratch(int device, hipStream_t s, void **out) {
  *out = nullptr;
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_ptr[device]) {
    // The caller has made `device` current.
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    const long long words = kNoAllocZeroBytes / 4;
    zero_words_kernel<<<dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s>>>(
        static_cast<unsigned *>(p), words);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    g_ptr[device] = p;
  }
  *out = g_ptr[device];
  return hipSuccess;
}

}  // namespace bnr
