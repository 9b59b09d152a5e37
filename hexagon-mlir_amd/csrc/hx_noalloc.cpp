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
// GPU shares its array: calls that overlap on one GPU race.  Nothing in it
// needs to start at zero (every kernel that reads a region writes all of it
// first in the same call), so no call clears it.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/hx.h"
#include "hx_api_internal.hpp"

static_assert(HX_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch size");

static __device__ __align__(256) char scratch[HX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices];  // per device, resolved once
}  // namespace

// Resolve the current device's scratch address (once per device).
int hx::noalloc_setup(char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return api_fail(HX_ERR_NODEVICE, "no HIP device visible");
  if (dev < 0 || dev >= kMaxDevices) return api_fail(HX_ERR_UNSUPPORTED, "device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return api_fail(HX_ERR_HIP, "scratch address on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<char*>(p);
  }
  if (out) *out = g_scratch_ptr[dev];
  return HX_OK;
}

extern "C" int hx_swiglu_ffn_noalloc(const hx_memref2d* x, const hx_memref1d* gamma, float eps,
                                     hx_weight_t w_gate, hx_weight_t w_up, hx_weight_t w_down, hx_memref2d* y,
                                     hx_stream_t stream) {
  char* base = nullptr;
  const int rc = hx::noalloc_setup(&base);
  if (rc) return rc;
  const hx::FixedScratch fs{base, (size_t)HX_NOALLOC_SCRATCH_BYTES};
  return hx::swiglu_ffn_impl(x, gamma, eps, w_gate, w_up, w_down, y, stream, &fs, "hx_swiglu_ffn_noalloc");
}
