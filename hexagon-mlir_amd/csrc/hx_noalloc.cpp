// hx_noalloc.cpp -- the entry point that allocates nothing:
// hx_swiglu_ffn_noalloc, the SwiGLU FFN block with every intermediate (the
// RMSNorm output, the gate/up products, the SiLU*mul activations) and the
// down projection's K-split partials held in a fixed per-GPU device array
// instead of the per-stream workspace.  It has no counterpart in the
// reference; it exists for callers that cannot call hipMalloc (code under
// HIP graph capture, tight serving loops, harnesses that forbid it).
//
// `scratch` below is a device variable: in host code its name is only a
// stand-in, so the library resolves each GPU's own copy once per device
// with hipGetSymbolAddress (at hx_init, or on the entry point's first call
// on that device) and passes that address to the kernels.  Every call on a
// GPU shares its array: calls that overlap on one GPU race.  Its last
// kGemvSplitCounters words are the split decode GEMV's counters, which must
// read zero when a call starts: the array is zero at load, a fill kernel
// clears them once when the device is set up (on the caller's stream, or
// synchronously at hx_init), and every kernel that counts on them returns
// them to zero.  Nothing else in it needs to start at zero (every kernel
// that reads a region writes all of it first in the same call).
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/hx.h"
#include "hx_api_internal.hpp"
#include "hx_internal.hpp"

static_assert(HX_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");
static constexpr size_t kCounterBytes = (size_t)hx::kGemvSplitCounters * sizeof(unsigned);
static_assert(kCounterBytes % 256 == 0 && kCounterBytes < HX_NOALLOC_SCRATCH_BYTES, "counter region");

static __device__ __align__(256) char scratch[HX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices];  // per device, resolved once
}  // namespace

// Resolve the current device's scratch address and clear its counters
// (once per device): on `s`, or with s == nullptr on the null stream and
// waited for.
int hx::noalloc_setup(char** out, unsigned** cnt, hipStream_t s) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return api_fail(HX_ERR_NODEVICE, "no HIP device visible");
  if (dev < 0 || dev >= kMaxDevices) return api_fail(HX_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return api_fail(HX_ERR_HIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
    unsigned* c = reinterpret_cast<unsigned*>(static_cast<char*>(p) + HX_NOALLOC_SCRATCH_BYTES - kCounterBytes);
    if (launch_fill_u32(c, kGemvSplitCounters, 0u, s) != HXI_OK || hipGetLastError() != hipSuccess ||
        (!s && hipStreamSynchronize(nullptr) != hipSuccess))
      return api_fail(HX_ERR_HIP, "clearing the scratch counters on device %d", dev);
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  if (out) *out = g_scratch_ptr[dev];
  if (cnt) *cnt = reinterpret_cast<unsigned*>(g_scratch_ptr[dev] + HX_NOALLOC_SCRATCH_BYTES - kCounterBytes);
  return HX_OK;
}

extern "C" int hx_swiglu_ffn_noalloc(const hx_memref2d* x, const hx_memref1d* gamma, float eps,
                                     hx_weight_t w_gate, hx_weight_t w_up, hx_weight_t w_down, hx_memref2d* y,
                                     hx_stream_t stream) {
  char* base = nullptr;
  unsigned* cnt = nullptr;
  const int rc = hx::noalloc_setup(&base, &cnt, (hipStream_t)stream);
  if (rc) return rc;
  const hx::FixedScratch fs{base, (size_t)HX_NOALLOC_SCRATCH_BYTES - kCounterBytes, cnt};
  return hx::swiglu_ffn_impl(x, gamma, eps, w_gate, w_up, w_down, y, stream, &fs, "hx_swiglu_ffn_noalloc");
}
