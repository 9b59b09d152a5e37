// hx_api_internal.hpp -- host-side helpers of the C ABI layer (hx_api.cpp)
// that the native autotuner (hx_tune.cpp) shares.  Nothing here is exported.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "../../include/hx.h"

namespace hx {

// Record `fmt` as the calling thread's hx_last_error() text; returns code.
int api_fail(int code, const char* fmt, ...);

// (gemm mode, epilogue) of a GEMM family; false for the GEMV families.
bool op_gemm(int op, int* mode, int* epi);
// The decode GEMV families (int8, f16, bf16 weights share one table).
bool gemv_op(int op);
// The row families (softmax, RMSNorm, LayerNorm): one shared table of row
// configurations, keyed (m, n, k) = (rows, cols, dtype).
bool row_family(int op);
// Table indices (into the mode's config table, or the GEMV table) of the
// configurations of family `op`, in family-index order.
std::vector<int> family_indices(int op);
// Family index of the untuned default configuration for this shape (the
// choice a call makes when nothing is pinned), -1 when that is the generic
// any-alignment kernel.
int untuned_family_index(int op, int64_t m, int64_t n, int64_t k);

// Canary references per (device, family): the median per-launch time of the
// fixed probe measured by the last valid tuning round (or loaded with the
// pins).  Returns false when none is held.
bool canary_reference_get(int dev, int op, double* q50_us);
void canary_reference_set(int dev, int op, double q50_us);
// Every (family, q50) held for a device, in family order.
std::vector<std::pair<int, double>> canary_references(int dev);

// Device memory a caller supplies so that a call allocates nothing.
struct FixedScratch {
  char* base;
  size_t cap;
  unsigned* cnt;  // kGemvSplitCounters counters of the split decode GEMV, zero between calls
};

// The current device's fixed scratch (hx_noalloc.cpp), resolved once per
// device; *out (may be null) receives its address.
int noalloc_setup(char** out, unsigned** cnt, hipStream_t s);

// The SwiGLU FFN block (hx_swiglu_ffn); with `fixed` every intermediate and
// K-split partial lives in that memory and the call allocates nothing.
int swiglu_ffn_impl(const hx_memref2d* x, const hx_memref1d* gamma, float eps, hx_weight_t w_gate,
                    hx_weight_t w_up, hx_weight_t w_down, hx_memref2d* y, hx_stream_t stream,
                    const FixedScratch* fixed, const char* entry);

}  // namespace hx
