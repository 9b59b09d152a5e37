// hx_api.cpp -- the C ABI of libhxmi (declared in include/hx.h): argument
// validation, the per-stream workspace, the resident-weight registry, the
// pinned-config table, and dispatch onto the kernel families.
//
// Ownership follows the reference runtime (QHB/bin/runtime/include/
// HexagonCAPI.h:21-68): callers own tensors, the library owns resident
// weights (hexagon_runtime_weight_resident_v2) and workspace
// (hexagon_runtime_workspace_resident_v2).  Unlike the reference, a failure
// returns a status instead of aborting, and resident weights are keyed by
// content, not by source address, so a changed weight is a new registration
// rather than a stale image (QHB/include/hexagon/Dialect/Hmx/Transforms/
// Passes.td:381-389 documents the reference's never-revalidated contents).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <atomic>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/hx.h"
#include "hx_api_internal.hpp"
#include "hx_device.hpp"
#include "hx_internal.hpp"

#ifndef HX_BUILD_ID
#define HX_BUILD_ID "hxmi-dev"
#endif

using namespace hx;

// ---------------------------------------------------------------------------
// Errors
// ---------------------------------------------------------------------------
static thread_local std::string g_err;

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hx::api_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

#define HX_HIP_TRY(expr)                                                              \
  do {                                                                                \
    hipError_t e_ = (expr);                                                           \
    if (e_ != hipSuccess) return fail(HX_ERR_HIP, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

static int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(HX_ERR_HIP, "%s launch: %s", what, hipGetErrorString(e));
  return HX_OK;
}

static int map_internal(int rc, const char* what) {
  if (rc == HXI_OK) return check_launch(what);
  switch (rc) {
    case HXI_ERR_UNSUPPORTED: return fail(HX_ERR_UNSUPPORTED, "%s: shape not supported", what);
    case HXI_ERR_DTYPE: return fail(HX_ERR_DTYPE, "%s: dtype not supported", what);
    case HXI_ERR_SHAPE: return fail(HX_ERR_SHAPE, "%s: bad shape", what);
    // set-up failures whose helper already recorded the message
    case HXI_ERR_NOMEM: return HX_ERR_NOMEM;
    case HXI_ERR_CAPTURE: return HX_ERR_UNSUPPORTED;
    default: return fail(HX_ERR_ARG, "%s: internal argument error %d", what, rc);
  }
}

// ---------------------------------------------------------------------------
// Device / workspace
// ---------------------------------------------------------------------------
static std::mutex g_mu;

static int current_device(int* dev) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return fail(HX_ERR_NODEVICE, "no HIP device visible");
  HX_HIP_TRY(hipGetDevice(dev));
  return HX_OK;
}

struct Workspace {
  char* buf = nullptr;  // carved by the top-level entry point of a call
  size_t bytes = 0;
};
static std::map<std::pair<int, hipStream_t>, Workspace> g_ws;

// A scratch region of at least `bytes` for work enqueued on `s`.  Growing it
// synchronizes `s` first, so kernels still reading the old region finish.
static int ws_get(hipStream_t s, size_t bytes, char** out) {
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_ws[{dev, s}];
  if (w.bytes < bytes) {
    size_t nb = bytes > 2 * w.bytes ? bytes : 2 * w.bytes;
    nb = (nb + 4095) & ~(size_t)4095;
    HX_HIP_TRY(hipStreamSynchronize(s));
    if (w.buf) HX_HIP_TRY(hipFree(w.buf));
    w.buf = nullptr;
    w.bytes = 0;
    if (hipMalloc(&w.buf, nb) != hipSuccess) return fail(HX_ERR_NOMEM, "workspace of %zu bytes", nb);
    w.bytes = nb;
  }
  *out = w.buf;
  return HX_OK;
}

// The binary32 partials of a K-split GEMM: a second per-stream region, so
// that growing it never moves the workspace a caller has already carved.
static std::map<std::pair<int, hipStream_t>, Workspace> g_part;
static int part_get(hipStream_t s, size_t bytes, float** out) {
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_part[{dev, s}];
  if (w.bytes < bytes) {
    size_t nb = (bytes + 4095) & ~(size_t)4095;
    HX_HIP_TRY(hipStreamSynchronize(s));
    if (w.buf) HX_HIP_TRY(hipFree(w.buf));
    w.buf = nullptr;
    w.bytes = 0;
    if (hipMalloc(&w.buf, nb) != hipSuccess) return fail(HX_ERR_NOMEM, "split-K partials of %zu bytes", nb);
    w.bytes = nb;
  }
  *out = reinterpret_cast<float*>(w.buf);
  return HX_OK;
}

// The K-split decode GEMV's buffers: its binary32 partials share the
// K-split GEMM's region (one kernel uses it at a time on a stream), and its
// per-group counters are a fixed region cleared once, when allocated, by a
// fill kernel on `s` followed by a wait for it (each kernel that counts
// returns the counters it used to zero).  Setting them up allocates and
// waits, so it cannot happen while `s` is being captured into a graph: the
// first split GEMV on a stream must run eagerly, and one captured before
// that is refused with HX_ERR_UNSUPPORTED rather than recording a clear that
// only a replay would run.
static std::map<std::pair<int, hipStream_t>, Workspace> g_cnt;
static int capture_refusal(hipStream_t s, const char* what) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &st) != hipSuccess) {
    (void)hipGetLastError();
    return fail(HX_ERR_HIP, "%s: querying the stream's capture status failed", what);
  }
  if (st != hipStreamCaptureStatusNone)
    return fail(HX_ERR_UNSUPPORTED,
                "%s: first use on this stream under graph capture (set-up allocates and waits; "
                "run one such call on the stream before capturing)", what);
  return HX_OK;
}
int hx::gemv_split_buffers(hipStream_t s, size_t part_bytes, float** part, unsigned** cnt) {
  int dev;
  if (current_device(&dev)) return HXI_ERR_NOMEM;
  bool ready;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    ready = g_cnt[{dev, s}].buf != nullptr && g_part[{dev, s}].bytes >= part_bytes;
  }
  if (!ready && capture_refusal(s, "split decode GEMV")) return HXI_ERR_CAPTURE;
  if (part_get(s, part_bytes, part)) return HXI_ERR_NOMEM;
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_cnt[{dev, s}];
  if (!w.buf) {
    const size_t nb = (size_t)kGemvSplitCounters * sizeof(unsigned);
    if (hipMalloc(&w.buf, nb) != hipSuccess) {
      w.buf = nullptr;
      fail(HX_ERR_NOMEM, "split GEMV counters of %zu bytes", nb);
      return HXI_ERR_NOMEM;
    }
    if (launch_fill_u32(reinterpret_cast<unsigned*>(w.buf), kGemvSplitCounters, 0u, s) != HXI_OK ||
        hipGetLastError() != hipSuccess || hipStreamSynchronize(s) != hipSuccess) {
      (void)hipFree(w.buf);
      w.buf = nullptr;
      fail(HX_ERR_NOMEM, "clearing the split GEMV counters");
      return HXI_ERR_NOMEM;
    }
    w.bytes = nb;
  }
  *cnt = reinterpret_cast<unsigned*>(w.buf);
  return HXI_OK;
}

// f32 operands quantised to f16 (hx_matmul): a third per-stream region, so
// that the workspace the f16 call then carves can grow without moving them.
static std::map<std::pair<int, hipStream_t>, Workspace> g_quant;
static int quant_get(hipStream_t s, size_t bytes, char** out) {
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_quant[{dev, s}];
  if (w.bytes < bytes) {
    size_t nb = (bytes + 4095) & ~(size_t)4095;
    HX_HIP_TRY(hipStreamSynchronize(s));
    if (w.buf) HX_HIP_TRY(hipFree(w.buf));
    w.buf = nullptr;
    w.bytes = 0;
    if (hipMalloc(&w.buf, nb) != hipSuccess) return fail(HX_ERR_NOMEM, "f32 operand quantisation of %zu bytes", nb);
    w.bytes = nb;
  }
  *out = w.buf;
  return HX_OK;
}

// Carve 256-byte aligned sub-buffers out of one workspace region.
struct Carver {
  size_t used = 0;
  size_t take(size_t bytes) {
    size_t at = used;
    used += (bytes + 255) & ~(size_t)255;
    return at;
  }
};

// ---------------------------------------------------------------------------
// Descriptors
// ---------------------------------------------------------------------------
static size_t dt_size(int dt) {
  switch (dt) {
    case HX_F16: case HX_BF16: return 2;
    case HX_F32: case HX_I32: return 4;
    case HX_I8: return 1;
    default: return 0;
  }
}
static const char* dt_name(int dt) {
  switch (dt) {
    case HX_F16: return "f16"; case HX_BF16: return "bf16"; case HX_F32: return "f32";
    case HX_I8: return "i8"; case HX_I32: return "i32"; default: return "?";
  }
}

struct View2 {
  char* p;
  int64_t rows, cols, ld;
};
struct View1 {
  char* p;
  int64_t n;
};

static int view2(const hx_memref2d* m, int dt, const char* name, View2* v) {
  if (!m) return fail(HX_ERR_ARG, "%s: null descriptor", name);
  const size_t es = dt_size(dt);
  if (!es) return fail(HX_ERR_DTYPE, "%s: unknown dtype %d", name, dt);
  if (m->sizes[0] < 0 || m->sizes[1] < 0 || m->offset < 0)
    return fail(HX_ERR_ARG, "%s: negative size/offset", name);
  v->rows = m->sizes[0];
  v->cols = m->sizes[1];
  if (v->rows > 0 && v->cols > 1 && m->strides[1] != 1)
    return fail(HX_ERR_LAYOUT, "%s: innermost stride %lld != 1", name, (long long)m->strides[1]);
  v->ld = m->strides[0];
  if (v->rows > 1 && v->ld < v->cols)
    return fail(HX_ERR_LAYOUT, "%s: row stride %lld < row length %lld", name, (long long)v->ld,
                (long long)v->cols);
  if (v->rows <= 1 && v->ld < v->cols) v->ld = v->cols;
  if (v->rows * v->cols > 0 && !m->aligned) return fail(HX_ERR_ARG, "%s: null data", name);
  v->p = (char*)m->aligned + m->offset * (int64_t)es;
  return HX_OK;
}

static int view1(const hx_memref1d* m, int dt, const char* name, int64_t expect, View1* v) {
  if (!m) return fail(HX_ERR_ARG, "%s: null descriptor", name);
  const size_t es = dt_size(dt);
  if (!es) return fail(HX_ERR_DTYPE, "%s: unknown dtype %d", name, dt);
  if (m->sizes[0] != expect)
    return fail(HX_ERR_SHAPE, "%s: length %lld, expected %lld", name, (long long)m->sizes[0],
                (long long)expect);
  if (m->sizes[0] > 1 && m->strides[0] != 1)
    return fail(HX_ERR_LAYOUT, "%s: stride %lld != 1", name, (long long)m->strides[0]);
  if (m->sizes[0] > 0 && !m->aligned) return fail(HX_ERR_ARG, "%s: null data", name);
  v->p = (char*)m->aligned + m->offset * (int64_t)es;
  v->n = m->sizes[0];
  return HX_OK;
}

// ---------------------------------------------------------------------------
// Plan manifest
// ---------------------------------------------------------------------------
// When enabled, every matmul-family call records the plan it ran: the kernel
// path, the tile configuration and whether it was pinned by the tuner or the
// untuned default, why the fast path was or was not taken, and how the weight
// was supplied.  One record per distinct decision, with a call count.  This
// is the run-time counterpart of the reference's per-matmul kernel manifest
// (plan + reason vocabulary, QHB/include/hexagon/Dialect/Hmx/Transforms/
// HmxManifest.h:81-110; its JSON export, QHB/backend/utils.py:1055-1196).
struct PlanCtx {
  const char* entry;   // C entry point the caller used
  const char* weight;  // "argument", "transposed-to-workspace", "resident-image", "resident-packed",
                       // "swapped-a-streamed" (N = 1: A streamed as the GEMV weight),
                       // "argument-kn" ([K][N] weight streamed in place)
  int a_dt, b_dt;
};

static std::atomic<int> g_manifest_on{0};
static std::mutex g_manifest_mu;
static std::vector<std::pair<std::string, uint64_t>> g_manifest;
static std::map<std::string, size_t> g_manifest_index;

static void note_plan(const PlanCtx& ctx, int64_t m, int64_t n, int64_t k, int c_dt, const char* plan,
                      const char* config, const char* source, const char* reason) {
  if (!g_manifest_on.load(std::memory_order_relaxed)) return;
  char rec[512];
  snprintf(rec, sizeof(rec),
           "{\"entry\": \"%s\", \"m\": %lld, \"n\": %lld, \"k\": %lld, \"a\": \"%s\", \"b\": \"%s\", "
           "\"c\": \"%s\", \"plan\": \"%s\", \"config\": \"%s\", \"config_source\": \"%s\", "
           "\"reason\": \"%s\", \"weight\": \"%s\"",
           ctx.entry, (long long)m, (long long)n, (long long)k, dt_name(ctx.a_dt), dt_name(ctx.b_dt),
           dt_name(c_dt), plan, config, source, reason, ctx.weight);
  std::lock_guard<std::mutex> lk(g_manifest_mu);
  auto it = g_manifest_index.find(rec);
  if (it != g_manifest_index.end()) {
    ++g_manifest[it->second].second;
    return;
  }
  g_manifest_index.emplace(rec, g_manifest.size());
  g_manifest.emplace_back(rec, 1);
}

extern "C" int hx_manifest_enable(int on) { return g_manifest_on.exchange(on ? 1 : 0); }

// ---------------------------------------------------------------------------
// Clock probe: three 64-bit counters per device (cycles, ticks, workgroups)
// that the tiled GEMM kernels add to while the probe is on.
// ---------------------------------------------------------------------------
static std::map<int, unsigned long long*> g_clk_buf;

extern "C" int hx_clock_probe(int enable) {
  int dev, rc;
  if ((rc = current_device(&dev))) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  unsigned long long*& buf = g_clk_buf[dev];
  if (!enable) {
    gemm_clock_target(dev, nullptr);
    return HX_OK;
  }
  if (!buf && hipMalloc(reinterpret_cast<void**>(&buf), 4 * sizeof(unsigned long long)) != hipSuccess) {
    buf = nullptr;
    return fail(HX_ERR_NOMEM, "hx_clock_probe: counters");
  }
  HX_HIP_TRY(hipDeviceSynchronize());
  HX_HIP_TRY(hipMemset(buf, 0, 4 * sizeof(unsigned long long)));
  HX_HIP_TRY(hipDeviceSynchronize());
  gemm_clock_target(dev, buf);
  return HX_OK;
}

extern "C" int hx_clock_read(double* mhz, double* workgroup_us, long long* workgroups) {
  int dev, rc;
  if ((rc = current_device(&dev))) return rc;
  unsigned long long* buf;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_clk_buf.find(dev);
    if (it == g_clk_buf.end() || !it->second) return fail(HX_ERR_ARG, "hx_clock_read: the probe was never enabled");
    buf = it->second;
  }
  unsigned long long h[3] = {0, 0, 0};
  HX_HIP_TRY(hipDeviceSynchronize());
  HX_HIP_TRY(hipMemcpy(h, buf, sizeof(h), hipMemcpyDeviceToHost));
  int khz = 0;
  HX_HIP_TRY(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  const double us = khz > 0 ? (double)h[1] / ((double)khz * 1e-3) : 0.0;  // ticks / (ticks per us)
  if (mhz) *mhz = us > 0 ? (double)h[0] / us : 0.0;
  if (workgroup_us) *workgroup_us = us;
  if (workgroups) *workgroups = (long long)h[2];
  return HX_OK;
}

extern "C" int hx_manifest_clear(void) {
  std::lock_guard<std::mutex> lk(g_manifest_mu);
  g_manifest.clear();
  g_manifest_index.clear();
  return HX_OK;
}

extern "C" int hx_manifest_json(char* buf, size_t cap, size_t* needed) {
  std::string out = "{\"schema\": \"hx.kernel_manifest/v1\", \"build\": \"" HX_BUILD_ID "\", \"records\": [";
  {
    std::lock_guard<std::mutex> lk(g_manifest_mu);
    for (size_t i = 0; i < g_manifest.size(); ++i) {
      if (i) out += ", ";
      out += g_manifest[i].first;
      out += ", \"calls\": " + std::to_string(g_manifest[i].second) + "}";
    }
  }
  out += "]}";
  if (needed) *needed = out.size() + 1;
  if (!buf || cap < out.size() + 1)
    return fail(HX_ERR_ARG, "hx_manifest_json: buffer of %zu bytes, %zu needed", cap, out.size() + 1);
  memcpy(buf, out.c_str(), out.size() + 1);
  return HX_OK;
}

// ---------------------------------------------------------------------------
// Pinned configurations
// ---------------------------------------------------------------------------
static std::map<std::tuple<int, int, int64_t, int64_t, int64_t>, int> g_pins;

// (gemm mode, epilogue) of each GEMM family
bool hx::op_gemm(int op, int* mode, int* epi) {
  switch (op) {
    case HX_OP_GEMM_I8: *mode = GM_I8; *epi = GE_STORE; return true;
    case HX_OP_MATMUL_F16: *mode = GM_F16; *epi = GE_STORE; return true;
    case HX_OP_MATMUL_BF16: *mode = GM_BF16; *epi = GE_STORE; return true;
    case HX_OP_MATMUL_W8: *mode = GM_W8; *epi = GE_STORE; return true;
    case HX_OP_SWIGLU_W8: *mode = GM_W8; *epi = GE_SWIGLU; return true;
    default: return false;
  }
}

// The decode GEMV families (int8, f16, bf16 weights) share one config table.
bool hx::gemv_op(int op) {
  return op == HX_OP_GEMV_W8 || op == HX_OP_GEMV_F16 || op == HX_OP_GEMV_BF16;
}

// The row families (softmax, RMSNorm, LayerNorm), keyed (rows, cols, dtype).
bool hx::row_family(int op) {
  return op == HX_OP_SOFTMAX || op == HX_OP_RMSNORM || op == HX_OP_LAYERNORM;
}

// Table indices (into the mode's table) of the configs of one family.
std::vector<int> hx::family_indices(int op) {
  std::vector<int> out;
  int mode, epi;
  if (row_family(op)) {
    for (int i = 0; i < row_config_count(); ++i) out.push_back(i);
    return out;
  }
  if (gemv_op(op)) {
    for (int i = 0; i < gemv_packed_config_count(); ++i) out.push_back(i);
    return out;
  }
  if (!op_gemm(op, &mode, &epi)) return out;
  for (int i = 0; i < gemm_config_count(mode); ++i)
    if (gemm_config(mode, i)->epi == epi) out.push_back(i);
  return out;
}

static int pinned(int op, int64_t m, int64_t n, int64_t k) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return -1;
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_pins.find(std::make_tuple(dev, op, m, n, k));
  return it == g_pins.end() ? -1 : it->second;
}

// Mode-table index a call of family `op` runs with (*was_pinned: chosen by
// the tuner rather than the untuned default).
static int resolve_gemm(int op, int64_t M, int64_t N, int64_t K, bool* was_pinned = nullptr) {
  int mode, epi;
  op_gemm(op, &mode, &epi);
  const int pin = pinned(op, M, N, K);
  if (was_pinned) *was_pinned = false;
  if (pin >= 0) {
    std::vector<int> idx = family_indices(op);
    if (pin < (int)idx.size()) {
      if (was_pinned) *was_pinned = true;
      return idx[pin];
    }
  }
  return gemm_default_config(mode, epi, M, N, K);
}
// Untuned GEMV config (table index = family index) for a shape.
// in_place: an [N][K] weight read where it lies (argument weights; f16 /
// bf16 have their own rules, int8 one of its own); otherwise a registered
// weight's packed image.
static int gemv_untuned_table(int op, int64_t M, int64_t N, int64_t K, bool in_place);
// The untuned config as it runs: a config that stages the activations in
// LDS, or splits K over workgroups, is named by its base config where the
// rows do not fit it (the launcher runs the base), so the tuner's control
// and the plan record match the kernel that runs.
static int gemv_untuned(int op, int64_t M, int64_t N, int64_t K, bool in_place = false) {
  const int t = gemv_untuned_table(op, M, N, K, in_place);
  const GemvConfig* c = gemv_packed_config(t);
  const int wt = op == HX_OP_GEMV_W8 ? HX_I8 : op == HX_OP_GEMV_BF16 ? HX_BF16 : HX_F16;
  return c && (!gemv_xl_fits(*c, M, K, wt) || (c->split > 1 && !gemv_split_takes(*c, M, N))) ? c->base : t;
}
static int gemv_untuned_table(int op, int64_t M, int64_t N, int64_t K, bool in_place) {
  if (M > 16) return gemv_rows_default(M, N, K);
  const int64_t tiles = (N + 15) / 16;
  const bool three_tiles = (tiles + 255) / 256 == 3;  // N = 11008: 688 tiles, 230 workgroups
  if (op != HX_OP_GEMV_W8 && in_place) {
    // f16 / bf16 weights in place, untuned choice from the MI355X sweep over
    // N, K in {4096, 8192, 11008}: 16 waves with LDS-staged activations for
    // M <= 2 (software pipelined once K spans several slices), 8 for M <= 4,
    // one column tile per workgroup (two for K >= 8192) beyond
    if (M <= 2) return K >= 8192 ? 12 : 7;
    if (M <= 4) return 5;
    return K >= 8192 ? 0 : 1;
  }
  if (op != HX_OP_GEMV_W8) {
    // the packed f16 / bf16 image: staged activations for M <= 4, over 16
    // or 8 waves.  M <= 2 from an interleaved A/B (five rounds, rotating
    // copies; M = 1, 16 against 8 waves, us): N = 4096 and K = 4096 / 8192 /
    // 11008 / 16384: 7.48 / 13.48 / 16.67 / 24.21 against 7.55 / 14.83 /
    // 16.69 / 23.27; N = 8192, K = 4096 / 8192: 13.50 / 23.66 against 12.69 /
    // 25.93; K = 4096, N = 11008 / 16384: 17.66 / 23.86 against 16.44 /
    // 21.85.  8 waves for M <= 4 otherwise; beyond, three tiles over 16 waves
    // where they give one workgroup per CU (16 x 11008 x 4096: 16.9 against
    // 24.7 us for one tile), two tiles from 512 tiles (16 x 8192 x 8192: 24.4
    // against 33.4) and one below (16 x 4096 x 16384: 30.6 against 39.5 for
    // two)
    if (M <= 2) return (K <= 4096 && tiles >= 512) || K >= 16384 ? 5 : 7;
    if (M <= 4) return 5;
    // K split over workgroups.  At most 128 tiles (one tile per workgroup
    // leaves half the CUs idle), K >= 8192: one tile over two parts up to 8
    // rows, two tiles over four beyond (M = 5 / 8 / 12 / 16 at 2048 x 8192:
    // 9.4 / 9.9 / 10.4 / 10.6 against 10.6 / 12.3 / 13.9 / 15.3 us unsplit;
    // 1024 x 8192: 8.3 / 9.0 / 9.0 / 9.4 against 10.1 / 11.7 / 11.8 / 12.7);
    // K = 4096 from 12 rows one tile over two parts (2048 x 4096: 7.4 / 7.7
    // against 8.0 / 8.8).  More than 8 rows with K >= 10240 on at most 256
    // tiles: two tiles over two parts (4096 x 11008, M = 9 / 12 / 16: 17.9 /
    // 18.4 / 19.3 against 18.4 / 20.0 / 22.1; at 4096 x 8192 the split lost,
    // 16.8 against 14.8 at M = 9).
    if (tiles <= 128 && K >= 8192) return M <= 8 ? 28 : 29;
    if (tiles <= 128 && K >= 4096 && M >= 12) return 28;
    // from 13 rows there four tiles over four parts with the loads issued
    // ahead (4096 x 11008, interleaved A/B, f16 / bf16 M = 9 / 12 / 14 / 16:
    // 18.11 / 18.26 / 18.43 / 18.61 and 18.92 / 18.38 / 18.51 / 18.67
    // against 17.79 / 18.33 / 18.81 / 19.24 and 18.73 / 18.34 / 18.77 /
    // 19.26 us for two tiles over two parts)
    if (M > 8 && tiles <= 256 && K >= 10240) return M > 12 ? 33 : 25;
    // one tile per workgroup issues its loads ahead (M = 8, f16 / bf16: 4096
    // x 4096 8.55 / 8.62 against 8.83 / 8.88 us, 4096 x 11008 17.62 / 18.03
    // against 18.00 / 18.18; at 16 rows 4096 x 4096 ties)
    return three_tiles ? 20 : tiles >= 512 ? 0 : 31;
  }
  // untuned choice from the MI355X sweep (int8, K = 4096).  When the
  // 16-column tiles need three per workgroup to fit one workgroup per CU
  // (N = 11008: 688 tiles, 230 workgroups): three tiles over 16 waves with
  // every slice load issued ahead of the MFMAs -- interleaved A/B, five
  // rounds on one box (bench.py --gemv-ab), M = 1 / 4 / 8 / 12 / 16: 9.40 /
  // 9.38 / 9.54 / 9.85 / 10.31 us, against 9.40 / 9.52 / 9.92 / 10.46 /
  // 11.07 for the compiler's load schedule and 9.67 / 9.60 / 9.82 / 10.00 /
  // 10.33 over 8 waves.  Otherwise, for M <= 4: up to 256 tiles one tile
  // per workgroup over 16 waves (M = 1 / 4, N = K = 4096: 5.19 / 5.30
  // against 5.24 / 5.38 issuing ahead, 5.50 / 5.63 with LDS-staged
  // activations over 8), beyond two tiles over 8 waves (M = 4, N = 8192 /
  // 16384: 7.67 / 12.73 against 8.15 / 13.97).
  // For M > 4 the fewest tiles per workgroup (1 to 4) that keep the
  // workgroups within one per CU, three beyond 1024 tiles (M = 16, N = 2048
  // / 4096 / 8192 / 16384 / 22016: 6.83 / 7.08 / 8.85 / 13.64 / 18.97 us;
  // four tiles everywhere took 9.63 / 9.86 / 10.5 / 13.64 / 22.25); one
  // tile issues its loads ahead (N = K = 4096, M = 8 / 16: 5.82 / 7.00
  // against 5.96 / 7.36; N = 4096, K = 11008, M = 8: 11.82 against 12.18).
  if (three_tiles) return 30;
  if (M <= 4) return tiles > 256 ? 0 : 24;
  // at most 128 tiles with K >= 8192, up to 12 rows: one tile per
  // workgroup over two parts (M = 5 / 8 / 12 at 2048 x 8192: 7.2 / 7.8 /
  // 8.4 against 7.7 / 8.6 / 8.8 us; 1024 x 8192: 7.0 / 7.6 / 8.3 against
  // 7.5 / 8.5 / 8.5).
  if (tiles <= 128 && K >= 8192 && M <= 12) return 28;
  // 12 rows or more on at most 256 tiles with K >= 8192: four tiles per
  // workgroup with K split over four workgroups, one workgroup per CU
  // (M = 12 / 16: 4096 x 11008 13.2 / 13.6 against 14.0 / 16.0 us; 2048 x
  // 8192 8.8 / 9.1 against 10.2 / 11.8; 4096 x 8192 10.3 / 10.5 against
  // 10.7 / 12.3; at M = 9 the split lost on N = 4096, 13.0 against 12.3),
  // its loads issued ahead (4096 x 11008: 13.07 / 13.40 against 13.24 /
  // 13.62 in the same A/B)
  if (M >= 12 && tiles <= 256 && K >= 8192) return 33;
  // an [N][K] weight read in place (sixteen 64-byte runs per wave load)
  // from 5 rows on at most 256 tiles with K >= 8192: the same split (M = 8,
  // 4096 x 11008: 16.13 us against 16.90 for ct1_kw8 and 19.44 for
  // ct1_kw8_e, which the packed image prefers)
  if (in_place && M > 4 && tiles <= 256 && K >= 8192) return 33;
  return tiles <= 256 ? 31 : tiles <= 512 ? 0 : tiles <= 768 ? 19 : tiles <= 1024 ? 10 : 19;
}

static int resolve_gemv(int op, int64_t M, int64_t N, int64_t K, bool* was_pinned = nullptr,
                        bool in_place = false) {
  const int pin = pinned(op, M, N, K);
  if (was_pinned) *was_pinned = pin >= 0 && pin < gemv_packed_config_count();
  if (pin >= 0 && pin < gemv_packed_config_count()) return pin;
  return gemv_untuned(op, M, N, K, in_place);
}

// RowOpCode of a row family.
static int row_op_code(int op) {
  return op == HX_OP_SOFTMAX ? ROW_OP_SOFTMAX : op == HX_OP_RMSNORM ? ROW_OP_RMSNORM : ROW_OP_LAYERNORM;
}

// Row configuration a call runs with: the pinned one, else the default.
static int resolve_row(int op, int64_t rows, int64_t cols, int dtype) {
  const int pin = pinned(op, rows, cols, dtype);
  if (pin >= 0 && pin < row_config_count()) return pin;
  return row_default_config(row_op_code(op), dtype, rows, cols);
}

int hx::untuned_family_index(int op, int64_t m, int64_t n, int64_t k) {
  if (row_family(op)) return row_default_config(row_op_code(op), (int)k, m, n);
  if (gemv_op(op)) return gemv_untuned(op, m, n, k);
  int mode, epi;
  if (!op_gemm(op, &mode, &epi)) return -1;
  const int t = gemm_default_config(mode, epi, m, n, k);
  const std::vector<int> idx = family_indices(op);
  for (size_t i = 0; i < idx.size(); ++i)
    if (idx[i] == t) return (int)i;
  return -1;
}

// Canary references of the tuner, per (device, family).
static std::map<std::pair<int, int>, double> g_canary;

bool hx::canary_reference_get(int dev, int op, double* q50_us) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_canary.find({dev, op});
  if (it == g_canary.end()) return false;
  *q50_us = it->second;
  return true;
}

void hx::canary_reference_set(int dev, int op, double q50_us) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_canary[{dev, op}] = q50_us;
}

std::vector<std::pair<int, double>> hx::canary_references(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::vector<std::pair<int, double>> out;
  for (const auto& kv : g_canary)
    if (kv.first.first == dev) out.emplace_back(kv.first.second, kv.second);
  return out;
}

// Where a K-split GEMM's binary32 partials go: the per-stream partials
// region (allocated on demand), or a caller-supplied buffer of `cap` bytes
// when the call must not allocate.
struct PartialsTarget {
  float* buf = nullptr;
  size_t cap = 0;
  bool fixed = false;
  unsigned* cnt = nullptr;  // the split decode GEMV's counters (fixed scratch)
};

// Partial bytes a run_gemm call of these args would need (0: no K split or
// not the tiled path).
static size_t gemm_partials_needed(int op, const GemmArgs& a) {
  int mode, epi;
  op_gemm(op, &mode, &epi);
  if (a.M == 0 || a.N == 0 || gemm_fast_refusal(mode, a)) return 0;
  const int cfg = resolve_gemm(op, a.M, a.N, a.K);
  return cfg >= 0 ? gemm_part_bytes(mode, cfg, a) : 0;
}

static int run_gemm(int op, GemmArgs& a, hipStream_t s, const PlanCtx& ctx,
                    const PartialsTarget& pt = PartialsTarget{}) {
  int mode, epi;
  op_gemm(op, &mode, &epi);
  if (a.M == 0 || a.N == 0) return HX_OK;
  const char* refusal = gemm_fast_refusal(mode, a);
  if (!refusal) {
    bool pin = false;
    const int cfg = resolve_gemm(op, a.M, a.N, a.K, &pin);
    if (cfg >= 0) {
      note_plan(ctx, a.M, a.N, a.K, a.out_dtype, "mfma-tiled", gemm_config(mode, cfg)->name,
                pin ? "pinned" : "default", "selected-aligned");
      if (const size_t pb = gemm_part_bytes(mode, cfg, a)) {
        // K split: partials, and the per-tile counters that let the last
        // part of each tile merge inside the kernel (the stream's split
        // counters, shared with the decode GEMV's split: kernels on one
        // stream run one at a time and leave them at zero)
        if (pt.fixed) {
          if (pb > pt.cap)
            return fail(HX_ERR_UNSUPPORTED, "%s: config %s needs %zu bytes of K-split partials, %zu reserved",
                        ctx.entry, gemm_config(mode, cfg)->name, pb, pt.cap);
          a.part = pt.buf;
          a.cnt = pt.cnt;
        } else {
          int rc = gemv_split_buffers(s, pb, &a.part, &a.cnt);
          if (rc) return map_internal(rc, "gemm split-K buffers");
        }
      }
      return map_internal(launch_gemm(mode, cfg, a, s), "gemm");
    }
    refusal = "no-config";
  }
  // the generic kernel reads B K-contiguous only (callers check the fast
  // path before passing a [K][N] B)
  if (a.b_kn) return fail(HX_ERR_UNSUPPORTED, "matmul: [K][N] B refused by the tiled kernel (%s)", refusal);
  note_plan(ctx, a.M, a.N, a.K, a.out_dtype, "mfma-generic", "generic_32x32", "fixed", refusal);
  return map_internal(launch_gemm_generic(mode, a, s), "gemm_generic");
}

// One activation row against an [N][K] matrix read in place, whole rows per
// wave (dt: the matrix's type).
static int run_rowdot(GemvArgs& a, int dt, const void* w, int64_t ldw, hipStream_t s, const PlanCtx& ctx,
                      const char* reason) {
  note_plan(ctx, a.M, a.N, a.K, dt == HX_BF16 ? HX_BF16 : HX_F16, "gemv-rowdot", "rowdot", "fixed", reason);
  return map_internal(launch_rowdot(dt, a, w, ldw, s), "rowdot");
}

// f16 / bf16 weights read in place from [N][K] by the streaming GEMV.
// dt: the weight's type (the output has the activations' type: bf16 for
// bf16 weights, else f16).
static int run_gemv_hw(GemvArgs& a, int dt, const void* w, int64_t ldw, hipStream_t s, const PlanCtx& ctx,
                       const char* reason = nullptr) {
  if (!reason) reason = a.M <= 16 ? "min-rows" : "few-rows";  // 16 < M: row-block configs
  const int op = dt == HX_BF16 ? HX_OP_GEMV_BF16 : dt == HX_I8 ? HX_OP_GEMV_W8 : HX_OP_GEMV_F16;
  bool pin = false;
  const int cfg = resolve_gemv(op, a.M, a.N, a.K, &pin, true);
  note_plan(ctx, a.M, a.N, a.K, dt == HX_BF16 ? HX_BF16 : HX_F16, "gemv-stream", gemv_packed_config(cfg)->name,
            pin ? "pinned" : "default", reason);
  return map_internal(launch_gemv_hw(cfg, dt, a, w, ldw, s), "gemv_stream");
}

static int run_gemv(GemvArgs& a, hipStream_t s, const PlanCtx& ctx) {
  static const char* const names[] = {"gemv_nk_ct1", "gemv_nk_ct2", "gemv_nk_ct4"};
  note_plan(ctx, a.M, a.N, a.K, HX_F16, "gemv", names[gemv_raw_config(a)], "fixed", "min-rows");
  return map_internal(launch_gemv_w8a16(a, s), "gemv_w8a16");
}

// ---------------------------------------------------------------------------
// Library state
// ---------------------------------------------------------------------------
extern "C" int hx_init(void) {
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  hipDeviceProp_t prop;
  HX_HIP_TRY(hipGetDeviceProperties(&prop, dev));
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(HX_ERR_UNSUPPORTED, "device %d is %s; libhxmi is built for gfx950 only", dev,
                prop.gcnArchName);
  // the no-allocation entry point's scratch address on this device
  return noalloc_setup(nullptr, nullptr, nullptr);
}

extern "C" const char* hx_last_error(void) { return g_err.c_str(); }
extern "C" const char* hx_build_id(void) { return HX_BUILD_ID; }

// ---------------------------------------------------------------------------
// Matmul family
// ---------------------------------------------------------------------------

// Bring B into the kernels' K-contiguous [N][K] form.  Returns the pointer
// and leading dimension to use; KN operands are transposed into `dst`.
static void* b_as_nk(const View2& b, int layout, size_t es, void* dst, int64_t* ld, hipStream_t s,
                     int* rc) {
  *rc = HX_OK;
  if (layout == HX_LAYOUT_NK) {
    *ld = b.ld;
    return b.p;
  }
  // b is [K][N] -> dst [N][K]
  int r = launch_transpose(b.p, b.ld, dst, b.rows, b.rows, b.cols, (int)es, s);
  *rc = map_internal(r, "transpose");
  *ld = b.rows;
  return dst;
}

static int scale_f32(const hx_memref1d* sc, int sdt, int64_t n, const char* name, float* dst,
                     const float** out, hipStream_t s) {
  *out = nullptr;
  if (!sc) return HX_OK;
  View1 v;
  int rc = view1(sc, sdt, name, n, &v);
  if (rc) return rc;
  if (sdt == HX_F32) {
    *out = (const float*)v.p;
    return HX_OK;
  }
  if (sdt != HX_F16) return fail(HX_ERR_DTYPE, "%s: scale dtype %s (f16 or f32)", name, dt_name(sdt));
  rc = map_internal(launch_f16_to_f32(v.p, dst, n, s), "scale widen");
  *out = dst;
  return rc;
}

extern "C" int hx_matmul(const hx_memref2d* a, int a_dtype, const hx_memref2d* b, int b_dtype,
                         int b_layout, const hx_memref1d* col_scale, int scale_dtype,
                         const hx_memref2d* residual, int residual_dtype, hx_memref2d* c,
                         int c_dtype, hx_stream_t stream) {
  hipStream_t s = (hipStream_t)stream;
  if (a_dtype == HX_F32 || (b_dtype == HX_F32 && (a_dtype == HX_F16 || a_dtype == HX_F32))) {
    // f32 operands are quantised to f16 as the reference's f32 pack does
    // ((x + 0) rounded to nearest even, -0 -> +0; QHB/bin/runtime/hmx/src/
    // HMXLayout.c:257-340), then multiplied on the f16 path with binary32
    // accumulation.  f32 A goes with an f16, f32 or int8 B; f32 B with f16
    // or f32 A.
    if (a_dtype == HX_F32 && b_dtype != HX_F32 && b_dtype != HX_F16 && b_dtype != HX_I8)
      return fail(HX_ERR_DTYPE, "hx_matmul: a=f32 with b=%s (f32, f16 or i8)", dt_name(b_dtype));
    View2 qa, qb;
    int rc;
    if ((rc = view2(a, a_dtype, "a", &qa)) || (rc = view2(b, b_dtype, "b", &qb))) return rc;
    Carver cv;
    const size_t off_qa = a_dtype == HX_F32 ? cv.take((size_t)qa.rows * qa.cols * 2) : 0;
    const size_t off_qb = b_dtype == HX_F32 ? cv.take((size_t)qb.rows * qb.cols * 2) : 0;
    char* q = nullptr;
    if (cv.used && (rc = quant_get(s, cv.used, &q))) return rc;
    hx_memref2d a16 = *a, b16 = *b;
    if (a_dtype == HX_F32) {
      rc = map_internal(launch_f32_to_f16_rne((const float*)qa.p, qa.ld, (uint16_t*)(q + off_qa), qa.rows, qa.cols, s),
                        "f32 quantisation");
      if (rc) return rc;
      a16 = hx_memref2d{q + off_qa, q + off_qa, 0, {qa.rows, qa.cols}, {qa.cols, 1}};
    }
    if (b_dtype == HX_F32) {
      rc = map_internal(launch_f32_to_f16_rne((const float*)qb.p, qb.ld, (uint16_t*)(q + off_qb), qb.rows, qb.cols, s),
                        "f32 quantisation");
      if (rc) return rc;
      b16 = hx_memref2d{q + off_qb, q + off_qb, 0, {qb.rows, qb.cols}, {qb.cols, 1}};
    }
    return hx_matmul(&a16, a_dtype == HX_F32 ? HX_F16 : a_dtype, &b16, b_dtype == HX_F32 ? HX_F16 : b_dtype,
                     b_layout, col_scale, scale_dtype, residual, residual_dtype, c, c_dtype, stream);
  }
  int op;
  if (a_dtype == HX_F16 && b_dtype == HX_F16) op = HX_OP_MATMUL_F16;
  else if (a_dtype == HX_BF16 && b_dtype == HX_BF16) op = HX_OP_MATMUL_BF16;
  else if (a_dtype == HX_F16 && b_dtype == HX_I8) op = HX_OP_MATMUL_W8;
  else return fail(HX_ERR_DTYPE, "hx_matmul: a=%s b=%s (f16.f16, bf16.bf16, f16.i8, or f32 with f16/f32/i8)",
                   dt_name(a_dtype), dt_name(b_dtype));
  if (c_dtype != HX_F16 && c_dtype != HX_BF16 && c_dtype != HX_F32)
    return fail(HX_ERR_DTYPE, "hx_matmul: c dtype %s", dt_name(c_dtype));
  if (b_layout != HX_LAYOUT_KN && b_layout != HX_LAYOUT_NK) return fail(HX_ERR_ARG, "hx_matmul: b_layout");
  View2 va, vb, vc, vr{};
  int rc;
  if ((rc = view2(a, a_dtype, "a", &va))) return rc;
  if ((rc = view2(b, b_dtype, "b", &vb))) return rc;
  if ((rc = view2(c, c_dtype, "c", &vc))) return rc;
  const int64_t M = va.rows, K = va.cols;
  const int64_t N = b_layout == HX_LAYOUT_KN ? vb.cols : vb.rows;
  const int64_t Kb = b_layout == HX_LAYOUT_KN ? vb.rows : vb.cols;
  if (Kb != K) return fail(HX_ERR_SHAPE, "hx_matmul: a is [%lld,%lld] but b has K=%lld", (long long)M, (long long)K, (long long)Kb);
  if (vc.rows != M || vc.cols != N)
    return fail(HX_ERR_SHAPE, "hx_matmul: c is [%lld,%lld], expected [%lld,%lld]", (long long)vc.rows,
                (long long)vc.cols, (long long)M, (long long)N);
  if (residual) {
    if (residual_dtype != HX_F16 && residual_dtype != HX_BF16 && residual_dtype != HX_F32)
      return fail(HX_ERR_DTYPE, "hx_matmul: residual dtype %s", dt_name(residual_dtype));
    if ((rc = view2(residual, residual_dtype, "residual", &vr))) return rc;
    if (vr.rows != M || vr.cols != N) return fail(HX_ERR_SHAPE, "hx_matmul: residual shape");
  }
  if (M == 0 || N == 0) return HX_OK;

  // N = 1 (a matrix-vector product, the reference tuner's (M, K, 1) rows):
  // C^T = b^T . A^T is the decode GEMV with the [M][K] operand A streamed as
  // its K-contiguous weight and b as the single activation row, when b and C
  // are contiguous vectors.  The tiled GEMM would pad N to 32.
  if (N == 1 && M > 16 && op != HX_OP_MATMUL_W8 && !residual && !col_scale && c_dtype == a_dtype &&
      (b_layout == HX_LAYOUT_NK || vb.ld == 1) && vc.ld == 1) {
    GemvArgs v{};
    v.x = vb.p; v.ldx = K; v.w = nullptr; v.ldw = 0;
    v.scale = nullptr; v.y = vc.p; v.ldy = M; v.M = 1; v.N = M; v.K = K;
    if (!rowdot_refusal(a_dtype, v, va.p, va.ld))
      return run_rowdot(v, a_dtype, va.p, va.ld, s, PlanCtx{"hx_matmul", "swapped-a-streamed", a_dtype, b_dtype},
                        "n-is-one");
    if (!gemv_hw_refusal(a_dtype, v, va.p, va.ld))
      return run_gemv_hw(v, a_dtype, va.p, va.ld, s, PlanCtx{"hx_matmul", "swapped-a-streamed", a_dtype, b_dtype},
                         "n-is-one");
  }

  // The decode GEMV epilogues read an f16 or f32 column scale directly (the
  // GEMM path widens an f16 scale into the workspace first).
  const float* sc32 = nullptr;
  const uint16_t* sc16 = nullptr;
  if (col_scale) {
    if (scale_dtype != HX_F16 && scale_dtype != HX_F32)
      return fail(HX_ERR_DTYPE, "col_scale: dtype %s (f16 or f32)", dt_name(scale_dtype));
    View1 vs;
    if ((rc = view1(col_scale, scale_dtype, "col_scale", N, &vs))) return rc;
    if (scale_dtype == HX_F16) sc16 = (const uint16_t*)vs.p;
    else sc32 = (const float*)vs.p;
  }
  // Argument weights: the decode GEMV for M <= 16, its row blocks up to
  // kGemvRowsMaxM rows for a K-contiguous weight of 2048..4096 columns; the
  // tiled GEMM (K split) beyond.  Measured with argument f16 weights
  // (K = 4096, rotating copies): at M = 17 / 32 the row blocks take 12.2 /
  // 15.8 us at N = 4096 against 18.4 tiled, and 29.7 / 29.8 at N = 11008
  // against 23.0 / 23.5 (the in-place read streams slower than a packed
  // image); with a [K][N] weight they lose (transposed first: 25.1 against
  // 14.0 at M = 17); below N = 2048 the tiled GEMM wins by up to 3x (64 x
  // 256 x 8192: 14.2 against 37.1).
  const bool gemv_rows = (M <= 16 || (gemv_rows_route(M, N, false) && b_layout == HX_LAYOUT_NK)) &&
                         M <= kGemvMaxRows && !residual && c_dtype == (op == HX_OP_MATMUL_W8 ? HX_F16 : a_dtype);

  // Decode shapes with weights in the [K][N] orientation: stream the weight
  // in place rather than transposing it into the workspace.
  if (b_layout == HX_LAYOUT_KN && M <= 16 && gemv_rows) {
    GemvArgs v{};
    v.x = va.p; v.ldx = va.ld; v.w = nullptr; v.ldw = 0;
    v.y = vc.p; v.ldy = vc.ld; v.M = M; v.N = N; v.K = K;
    v.scale = sc32; v.scale16 = sc16;
    if (!gemv_kn_refusal(b_dtype, v, vb.p, vb.ld)) {
      const int parts = gemv_kn_parts(b_dtype, v);
      Carver kv;
      const size_t off_part = kv.take(gemv_kn_part_bytes(v, parts));
      char* ws = nullptr;
      if (kv.used && (rc = ws_get(s, kv.used, &ws))) return rc;
      note_plan(PlanCtx{"hx_matmul", "argument-kn", a_dtype, b_dtype}, M, N, K, c_dtype, "gemv-kn",
                parts > 1 ? "kn_split" : "kn", "fixed", "min-rows");
      return map_internal(launch_gemv_kn(b_dtype, v, vb.p, vb.ld, parts, parts > 1 ? (float*)(ws + off_part) : nullptr, s),
                          "gemv_kn");
    }
  }

  // Decode shapes with a K-contiguous [N][K] weight: the streaming GEMV reads
  // it in place (the older 4-wave int8 kernel covers what it refuses).
  if (b_layout == HX_LAYOUT_NK && gemv_rows) {
    const PlanCtx nctx{"hx_matmul", "argument", a_dtype, b_dtype};
    GemvArgs v{};
    v.x = va.p; v.ldx = va.ld; v.w = (const int8_t*)vb.p; v.ldw = vb.ld;
    v.scale = sc32; v.scale16 = sc16; v.y = vc.p; v.ldy = vc.ld; v.M = M; v.N = N; v.K = K;
    if (M == 1 && !rowdot_refusal(b_dtype, v, vb.p, vb.ld)) return run_rowdot(v, b_dtype, vb.p, vb.ld, s, nctx, "one-row");
    if (!gemv_hw_refusal(b_dtype, v, vb.p, vb.ld)) return run_gemv_hw(v, b_dtype, vb.p, vb.ld, s, nctx);
    if (op == HX_OP_MATMUL_W8 && M <= 16 && gemv_fast_ok(v)) return run_gemv(v, s, nctx);
  }

  // [K][N] f16 / bf16 operands beyond the decode GEMV's rows: the tiled
  // kernel reads B in place (transposing LDS reads) when its fast path takes
  // the shape; otherwise B is transposed into the workspace.
  bool kn_native = false;
  if (b_layout == HX_LAYOUT_KN && (op == HX_OP_MATMUL_F16 || op == HX_OP_MATMUL_BF16) && !gemv_rows) {
    int mode, epi;
    op_gemm(op, &mode, &epi);
    GemmArgs t{};
    t.a = va.p; t.lda = va.ld; t.b = vb.p; t.ldb = vb.ld; t.c = vc.p; t.ldc = vc.ld;
    t.M = M; t.N = N; t.K = K; t.b_kn = 1;
    if (residual) { t.res = vr.p; t.ldr = vr.ld; t.res_dtype = residual_dtype; }
    kn_native = gemm_fast_refusal(mode, t) == nullptr;
  }

  const size_t eb = dt_size(b_dtype);
  Carver cv;
  const size_t off_bt = (b_layout == HX_LAYOUT_KN && !kn_native) ? cv.take((size_t)N * K * eb) : 0;
  const size_t off_sc = (col_scale && scale_dtype == HX_F16) ? cv.take((size_t)N * 4) : 0;
  char* ws = nullptr;
  if (cv.used && (rc = ws_get(s, cv.used, &ws))) return rc;

  GemmArgs g{};
  g.a = va.p; g.lda = va.ld;
  if (kn_native) {
    g.b = vb.p; g.ldb = vb.ld; g.b_kn = 1;
  } else {
    g.b = b_as_nk(vb, b_layout, eb, ws + off_bt, &g.ldb, s, &rc);
    if (rc) return rc;
  }
  g.c = vc.p; g.ldc = vc.ld;
  g.M = M; g.N = N; g.K = K;
  g.out_dtype = c_dtype;
  if ((rc = scale_f32(col_scale, scale_dtype, N, "col_scale", (float*)(ws + off_sc), &g.col_scale, s)))
    return rc;
  if (residual) { g.res = vr.p; g.ldr = vr.ld; g.res_dtype = residual_dtype; }

  const PlanCtx ctx{"hx_matmul",
                    kn_native ? "argument-kn" : b_layout == HX_LAYOUT_KN ? "transposed-to-workspace" : "argument",
                    a_dtype, b_dtype};
  // [K][N] weights the in-place GEMV refused: the transposed copy
  if (b_layout == HX_LAYOUT_KN && gemv_rows && !kn_native) {
    GemvArgs v{};
    v.x = g.a; v.ldx = g.lda; v.w = (const int8_t*)g.b; v.ldw = g.ldb;
    v.scale = g.col_scale; v.y = g.c; v.ldy = g.ldc; v.M = M; v.N = N; v.K = K;
    if (!gemv_hw_refusal(b_dtype, v, g.b, g.ldb)) return run_gemv_hw(v, b_dtype, g.b, g.ldb, s, ctx);
    if (op == HX_OP_MATMUL_W8 && M <= 16 && gemv_fast_ok(v)) return run_gemv(v, s, ctx);
  }
  return run_gemm(op, g, s, ctx);
}

extern "C" int hx_gemm_i8(const hx_memref2d* a, const hx_memref2d* b, int b_layout,
                          const hx_memref1d* row_scale, const hx_memref1d* col_scale,
                          hx_memref2d* c, int c_dtype, hx_stream_t stream) {
  hipStream_t s = (hipStream_t)stream;
  if (c_dtype != HX_I32 && c_dtype != HX_F16 && c_dtype != HX_BF16 && c_dtype != HX_F32)
    return fail(HX_ERR_DTYPE, "hx_gemm_i8: c dtype %s", dt_name(c_dtype));
  if (b_layout != HX_LAYOUT_KN && b_layout != HX_LAYOUT_NK) return fail(HX_ERR_ARG, "hx_gemm_i8: b_layout");
  View2 va, vb, vc;
  int rc;
  if ((rc = view2(a, HX_I8, "a", &va))) return rc;
  if ((rc = view2(b, HX_I8, "b", &vb))) return rc;
  if ((rc = view2(c, c_dtype, "c", &vc))) return rc;
  const int64_t M = va.rows, K = va.cols;
  const int64_t N = b_layout == HX_LAYOUT_KN ? vb.cols : vb.rows;
  const int64_t Kb = b_layout == HX_LAYOUT_KN ? vb.rows : vb.cols;
  if (Kb != K) return fail(HX_ERR_SHAPE, "hx_gemm_i8: K mismatch %lld vs %lld", (long long)K, (long long)Kb);
  if (vc.rows != M || vc.cols != N) return fail(HX_ERR_SHAPE, "hx_gemm_i8: c shape");
  if (c_dtype == HX_I32 && (row_scale || col_scale))
    return fail(HX_ERR_ARG, "hx_gemm_i8: scales apply only to a floating output");
  View1 vrs{}, vcs{};
  if (row_scale && (rc = view1(row_scale, HX_F32, "row_scale", M, &vrs))) return rc;
  if (col_scale && (rc = view1(col_scale, HX_F32, "col_scale", N, &vcs))) return rc;
  if (M == 0 || N == 0) return HX_OK;

  GemmArgs g{};
  g.a = va.p; g.lda = va.ld;
  g.c = vc.p; g.ldc = vc.ld;
  g.M = M; g.N = N; g.K = K;
  g.out_dtype = c_dtype;
  g.row_scale = row_scale ? (const float*)vrs.p : nullptr;
  g.col_scale = col_scale ? (const float*)vcs.p : nullptr;
  // a [K][N] B is read in place by the tiled kernel (transposing LDS reads)
  // when its fast path takes the shape, else transposed into the workspace.
  // The in-place main loop issues twice the B read instructions (8-byte
  // transposing reads) and runs about 20% slower than on a [N][K] B (74
  // against 61 us at 4096^3), which the transpose it replaces costs as well
  // (74.4 us for transpose + GEMM), without the N K bytes of workspace.
  bool kn_native = false;
  if (b_layout == HX_LAYOUT_KN) {
    GemmArgs t = g;
    t.b = vb.p; t.ldb = vb.ld; t.b_kn = 1;
    kn_native = gemm_fast_refusal(GM_I8, t) == nullptr;
  }
  if (kn_native) {
    g.b = vb.p; g.ldb = vb.ld; g.b_kn = 1;
  } else {
    Carver cv;
    const size_t off_bt = b_layout == HX_LAYOUT_KN ? cv.take((size_t)N * K) : 0;
    char* ws = nullptr;
    if (cv.used && (rc = ws_get(s, cv.used, &ws))) return rc;
    g.b = b_as_nk(vb, b_layout, 1, ws + off_bt, &g.ldb, s, &rc);
    if (rc) return rc;
  }
  const PlanCtx ctx{"hx_gemm_i8",
                    kn_native ? "argument-kn" : b_layout == HX_LAYOUT_KN ? "transposed-to-workspace" : "argument",
                    HX_I8, HX_I8};
  return run_gemm(HX_OP_GEMM_I8, g, s, ctx);
}

extern "C" int hx_gemv_w8a16(const hx_memref2d* x, const hx_memref2d* w, int w_layout,
                             const hx_memref1d* scale, int scale_dtype, hx_memref2d* y,
                             hx_stream_t stream) {
  return hx_matmul(x, HX_F16, w, HX_I8, w_layout, scale, scale_dtype, nullptr, 0, y, HX_F16, stream);
}

// ---------------------------------------------------------------------------
// Row reductions
// ---------------------------------------------------------------------------
static int row_dtype_ok(int dt, const char* who) {
  if (dt != HX_F16 && dt != HX_BF16 && dt != HX_F32)
    return fail(HX_ERR_DTYPE, "%s: dtype %s (f16, bf16 or f32)", who, dt_name(dt));
  return HX_OK;
}

// A row longer than the register path holds: the two-pass kernels, their
// per-segment statistics in the stream's workspace.
static int run_row_long(int op, int dtype, const View2& vx, const void* w, const void* b, float eps,
                        const View2& vy, float* mean, float* rstd, hipStream_t s, const char* what) {
  char* ws = nullptr;
  int rc = ws_get(s, row_long_ws_bytes(dtype, vx.rows, vx.cols), &ws);
  if (rc) return rc;
  return map_internal(launch_row_long(op, dtype, vx.p, vx.ld, w, b, eps, vy.p, vy.ld, mean, rstd, vx.rows,
                                      vx.cols, ws, s),
                      what);
}

extern "C" int hx_softmax(const hx_memref2d* x, hx_memref2d* y, int dtype, hx_stream_t stream) {
  int rc;
  if ((rc = row_dtype_ok(dtype, "hx_softmax"))) return rc;
  View2 vx, vy;
  if ((rc = view2(x, dtype, "x", &vx)) || (rc = view2(y, dtype, "y", &vy))) return rc;
  if (vx.rows != vy.rows || vx.cols != vy.cols) return fail(HX_ERR_SHAPE, "hx_softmax: x/y shape");
  if (vx.rows == 0 || vx.cols == 0) return HX_OK;
  const hipStream_t s = (hipStream_t)stream;
  rc = launch_softmax(dtype, vx.p, vx.ld, vy.p, vy.ld, vx.rows, vx.cols, s,
                      resolve_row(HX_OP_SOFTMAX, vx.rows, vx.cols, dtype));
  if (rc == HXI_ERR_UNSUPPORTED)
    return run_row_long(ROW_OP_SOFTMAX, dtype, vx, nullptr, nullptr, 0.f, vy, nullptr, nullptr, s, "softmax");
  return map_internal(rc, "softmax");
}

extern "C" int hx_rmsnorm(const hx_memref2d* x, const hx_memref1d* gamma, float eps, hx_memref2d* y,
                          int dtype, hx_stream_t stream) {
  int rc;
  if ((rc = row_dtype_ok(dtype, "hx_rmsnorm"))) return rc;
  View2 vx, vy;
  View1 vg{};
  if ((rc = view2(x, dtype, "x", &vx)) || (rc = view2(y, dtype, "y", &vy))) return rc;
  if (vx.rows != vy.rows || vx.cols != vy.cols) return fail(HX_ERR_SHAPE, "hx_rmsnorm: x/y shape");
  if (gamma && (rc = view1(gamma, dtype, "gamma", vx.cols, &vg))) return rc;
  if (vx.rows == 0 || vx.cols == 0) return HX_OK;
  const hipStream_t s = (hipStream_t)stream;
  rc = launch_rmsnorm(dtype, vx.p, vx.ld, gamma ? vg.p : nullptr, eps, vy.p, vy.ld, vx.rows, vx.cols, s,
                      resolve_row(HX_OP_RMSNORM, vx.rows, vx.cols, dtype));
  if (rc == HXI_ERR_UNSUPPORTED)
    return run_row_long(ROW_OP_RMSNORM, dtype, vx, gamma ? vg.p : nullptr, nullptr, eps, vy, nullptr, nullptr, s,
                        "rmsnorm");
  return map_internal(rc, "rmsnorm");
}

extern "C" int hx_layernorm(const hx_memref2d* x, const hx_memref1d* w, const hx_memref1d* b, float eps,
                            hx_memref2d* y, hx_memref1d* mean, hx_memref1d* rstd, int dtype,
                            hx_stream_t stream) {
  int rc;
  if ((rc = row_dtype_ok(dtype, "hx_layernorm"))) return rc;
  View2 vx, vy;
  View1 vw{}, vb{}, vm{}, vr{};
  if ((rc = view2(x, dtype, "x", &vx)) || (rc = view2(y, dtype, "y", &vy))) return rc;
  if (vx.rows != vy.rows || vx.cols != vy.cols) return fail(HX_ERR_SHAPE, "hx_layernorm: x/y shape");
  if (w && (rc = view1(w, dtype, "w", vx.cols, &vw))) return rc;
  if (b && (rc = view1(b, dtype, "b", vx.cols, &vb))) return rc;
  if (mean && (rc = view1(mean, HX_F32, "mean", vx.rows, &vm))) return rc;
  if (rstd && (rc = view1(rstd, HX_F32, "rstd", vx.rows, &vr))) return rc;
  if (vx.rows == 0 || vx.cols == 0) return HX_OK;
  const hipStream_t s = (hipStream_t)stream;
  float* mp = mean ? (float*)vm.p : nullptr;
  float* rp = rstd ? (float*)vr.p : nullptr;
  rc = launch_layernorm(dtype, vx.p, vx.ld, w ? vw.p : nullptr, b ? vb.p : nullptr, eps, vy.p, vy.ld, mp, rp,
                        vx.rows, vx.cols, s, resolve_row(HX_OP_LAYERNORM, vx.rows, vx.cols, dtype));
  if (rc == HXI_ERR_UNSUPPORTED)
    return run_row_long(ROW_OP_LAYERNORM, dtype, vx, w ? vw.p : nullptr, b ? vb.p : nullptr, eps, vy, mp, rp, s,
                        "layernorm");
  return map_internal(rc, "layernorm");
}

extern "C" int hx_silu_mul(const hx_memref2d* g, const hx_memref2d* u, hx_memref2d* out, int dtype,
                           hx_stream_t stream) {
  if (dtype != HX_F16) return fail(HX_ERR_DTYPE, "hx_silu_mul: f16 only");
  int rc;
  View2 vg, vu, vo;
  if ((rc = view2(g, dtype, "g", &vg)) || (rc = view2(u, dtype, "u", &vu)) || (rc = view2(out, dtype, "out", &vo)))
    return rc;
  if (vg.rows != vu.rows || vg.cols != vu.cols || vg.rows != vo.rows || vg.cols != vo.cols)
    return fail(HX_ERR_SHAPE, "hx_silu_mul: shapes differ");
  if (vg.rows == 0 || vg.cols == 0) return HX_OK;
  return map_internal(launch_silu_mul_f16(vg.p, vg.ld, vu.p, vu.ld, vo.p, vo.ld, vg.rows, vg.cols,
                                          (hipStream_t)stream),
                      "silu_mul");
}

// ---------------------------------------------------------------------------
// Attention
// ---------------------------------------------------------------------------
static int view4(const hx_memref4d* m, const char* name, const int64_t* expect, int64_t* strides,
                 const char** base) {
  if (!m) return fail(HX_ERR_ARG, "%s: null descriptor", name);
  for (int i = 0; i < 4; ++i) {
    if (m->sizes[i] < 0) return fail(HX_ERR_ARG, "%s: negative size", name);
    if (expect[i] >= 0 && m->sizes[i] != expect[i])
      return fail(HX_ERR_SHAPE, "%s: dim %d is %lld, expected %lld", name, i, (long long)m->sizes[i],
                  (long long)expect[i]);
  }
  if (m->sizes[3] > 1 && m->strides[3] != 1)
    return fail(HX_ERR_LAYOUT, "%s: innermost stride %lld != 1", name, (long long)m->strides[3]);
  if (m->offset < 0) return fail(HX_ERR_ARG, "%s: negative offset", name);
  const int64_t n = m->sizes[0] * m->sizes[1] * m->sizes[2] * m->sizes[3];
  if (n > 0 && !m->aligned) return fail(HX_ERR_ARG, "%s: null data", name);
  for (int i = 0; i < 3; ++i) strides[i] = m->strides[i];
  *base = (const char*)m->aligned + m->offset * 2;
  return HX_OK;
}

extern "C" int hx_attention(const hx_memref4d* q, const hx_memref4d* k, const hx_memref4d* v,
                            hx_memref4d* o, float scale, int causal, int dtype, hx_stream_t stream) {
  if (dtype != HX_F16 && dtype != HX_BF16)
    return fail(HX_ERR_DTYPE, "hx_attention: dtype %s (f16 or bf16)", dt_name(dtype));
  if (!q || !k) return fail(HX_ERR_ARG, "hx_attention: null descriptor");
  const int64_t Z = q->sizes[0], H = q->sizes[1], Nq = q->sizes[2], D = q->sizes[3];
  const int64_t Nk = k->sizes[2];
  AttnArgs a{};
  const char *bq, *bk, *bv, *bo;
  int rc;
  const int64_t eq[4] = {Z, H, Nq, D}, ek[4] = {Z, H, Nk, D};
  if ((rc = view4(q, "q", eq, a.sq, &bq)) || (rc = view4(k, "k", ek, a.sk, &bk)) ||
      (rc = view4(v, "v", ek, a.sv, &bv)) || (rc = view4(o, "o", eq, a.so, &bo)))
    return rc;
  a.q = bq; a.k = bk; a.v = bv; a.o = (void*)bo;
  a.Z = Z; a.H = H; a.Nq = Nq; a.Nk = Nk; a.D = D;
  a.scale = scale;
  a.causal_offset = 0;
  if (Z == 0 || H == 0 || Nq == 0) return HX_OK;
  if (const char* why = attn_refusal(a))
    return fail(HX_ERR_UNSUPPORTED, "hx_attention: %s (D=%lld; D must be 64 or 128, bases 16-byte "
                "aligned, strides multiples of 8)", why, (long long)D);
  // few (head, query block) workgroups: split the key range, partials in
  // the stream's workspace
  a.splits = attn_splits(a);
  a.part = nullptr;
  if (a.splits > 1) {
    char* ws = nullptr;
    if ((rc = ws_get((hipStream_t)stream, attn_part_bytes(a), &ws))) return rc;
    a.part = reinterpret_cast<float*>(ws);
  }
  return map_internal(launch_attention(dtype, causal != 0, a, (hipStream_t)stream), "attention");
}

// ---------------------------------------------------------------------------
// Resident weights
// ---------------------------------------------------------------------------
struct hx_weight {
  int device;
  int64_t K, N;
  int dtype;
  void* image;     // [N][K], K-contiguous (the GEMM operand)
  void* packed;    // MFMA-fragment-ordered copy for the decode GEMV (int8: 16 x 64 bytes
                   // per KiB block, f16 / bf16: 16 x 32 halves)
  float* scale;    // [N] or null
  uint64_t hash;
  int refcount;    // registrations not yet released
  int inuse;       // entry-point calls currently holding the weight
};
static std::set<hx_weight*> g_weights;

// Free a weight no registration and no call holds any more.  The
// synchronization makes sure no enqueued kernel still reads the image.
static void weight_free(hx_weight* x) {
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(x->device);
  (void)hipDeviceSynchronize();
  (void)hipFree(x->image);
  if (x->packed) (void)hipFree(x->packed);
  if (x->scale) (void)hipFree(x->scale);
  (void)hipSetDevice(cur);
  delete x;
}

// Weights whose last holder was a call that may not free device memory
// (the no-allocation entry points); the next registration or release frees
// them.
static std::vector<hx_weight*> g_deferred;

static void free_deferred() {
  std::vector<hx_weight*> dead;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    dead.swap(g_deferred);
  }
  for (hx_weight* x : dead) weight_free(x);
}

// A weight held for the duration of one entry-point call: a release on
// another thread in the meantime only drops the registration, and the
// memory goes when the last holder lets go (or, for a call that may not
// free, at the next registration or release).
class WeightUse {
 public:
  explicit WeightUse(hx_weight_t w, bool may_free = true) : may_free_(may_free) {
    std::lock_guard<std::mutex> lk(g_mu);
    if (w && g_weights.count(w) && w->refcount > 0) {
      ++w->inuse;
      w_ = w;
    }
  }
  ~WeightUse() {
    if (!w_) return;
    bool last;
    {
      std::lock_guard<std::mutex> lk(g_mu);
      last = --w_->inuse == 0 && w_->refcount == 0;
      if (last) {
        g_weights.erase(w_);
        if (!may_free_) g_deferred.push_back(w_);
      }
    }
    if (last && may_free_) weight_free(w_);
  }
  WeightUse(const WeightUse&) = delete;
  WeightUse& operator=(const WeightUse&) = delete;
  hx_weight* get() const { return w_; }

 private:
  hx_weight* w_ = nullptr;
  bool may_free_;
};

extern "C" int hx_weight_register(const hx_memref2d* w, int w_dtype, int w_layout,
                                  const hx_memref1d* scale, int scale_dtype, hx_stream_t stream,
                                  hx_weight_t* out) {
  hipStream_t s = (hipStream_t)stream;
  if (!out) return fail(HX_ERR_ARG, "hx_weight_register: null out");
  free_deferred();
  *out = nullptr;
  if (w_dtype == HX_F32) {
    // an f32 weight is quantised to f16 first, as the reference's host
    // prepack does ((w + 0) rounded to nearest even, -0 -> +0;
    // QHB/backend/hmx_weight_prepack.py:185-212), and registered as f16
    View2 v;
    int rc = view2(w, HX_F32, "w", &v);
    if (rc) return rc;
    uint16_t* tmp = nullptr;
    if (v.rows * v.cols > 0 && hipMalloc((void**)&tmp, (size_t)v.rows * v.cols * 2) != hipSuccess)
      return fail(HX_ERR_NOMEM, "hx_weight_register: f32 quantisation buffer");
    rc = map_internal(launch_f32_to_f16_rne((const float*)v.p, v.ld, tmp, v.rows, v.cols, s), "f32 quantisation");
    if (!rc) {
      hx_memref2d w16{tmp, tmp, 0, {v.rows, v.cols}, {v.cols, 1}};
      rc = hx_weight_register(&w16, HX_F16, w_layout, scale, scale_dtype, stream, out);
    }
    // registration synchronized the stream: the f16 copy is no longer read
    (void)hipStreamSynchronize(s);
    if (tmp) (void)hipFree(tmp);
    return rc;
  }
  if (w_dtype != HX_I8 && w_dtype != HX_F16 && w_dtype != HX_BF16)
    return fail(HX_ERR_DTYPE, "hx_weight_register: dtype %s", dt_name(w_dtype));
  if (w_layout != HX_LAYOUT_KN && w_layout != HX_LAYOUT_NK) return fail(HX_ERR_ARG, "hx_weight_register: layout");
  if (w_dtype == HX_I8 && !scale) return fail(HX_ERR_ARG, "hx_weight_register: int8 weights need scales");
  int dev, rc;
  if ((rc = current_device(&dev))) return rc;
  View2 vw;
  if ((rc = view2(w, w_dtype, "w", &vw))) return rc;
  const int64_t K = w_layout == HX_LAYOUT_KN ? vw.rows : vw.cols;
  const int64_t N = w_layout == HX_LAYOUT_KN ? vw.cols : vw.rows;
  if (K <= 0 || N <= 0) return fail(HX_ERR_SHAPE, "hx_weight_register: empty weight");
  View1 vs{};
  if (scale && (rc = view1(scale, scale_dtype, "scale", N, &vs))) return rc;
  if (scale && scale_dtype != HX_F16 && scale_dtype != HX_F32)
    return fail(HX_ERR_DTYPE, "hx_weight_register: scale dtype %s", dt_name(scale_dtype));

  const size_t es = dt_size(w_dtype);
  void* image = nullptr;
  float* sc = nullptr;
  uint64_t* hdev = nullptr;
  auto cleanup = [&]() {
    if (image) (void)hipFree(image);
    if (sc) (void)hipFree(sc);
    if (hdev) (void)hipFree(hdev);
  };
  if (hipMalloc(&image, (size_t)N * K * es) != hipSuccess) { cleanup(); return fail(HX_ERR_NOMEM, "weight image"); }
  if (scale && hipMalloc((void**)&sc, (size_t)N * 4) != hipSuccess) { cleanup(); return fail(HX_ERR_NOMEM, "weight scale"); }
  if (hipMalloc((void**)&hdev, 16) != hipSuccess) { cleanup(); return fail(HX_ERR_NOMEM, "hash"); }
  hipError_t e;
  if (w_layout == HX_LAYOUT_KN) {
    rc = map_internal(launch_transpose(vw.p, vw.ld, image, K, K, N, (int)es, s), "transpose");
  } else {
    e = hipMemcpy2DAsync(image, K * es, vw.p, vw.ld * es, K * es, N, hipMemcpyDeviceToDevice, s);
    rc = e == hipSuccess ? HX_OK : fail(HX_ERR_HIP, "weight copy: %s", hipGetErrorString(e));
  }
  if (!rc && scale) {
    if (scale_dtype == HX_F16) rc = map_internal(launch_f16_to_f32(vs.p, sc, N, s), "scale widen");
    else {
      e = hipMemcpyAsync(sc, vs.p, (size_t)N * 4, hipMemcpyDeviceToDevice, s);
      rc = e == hipSuccess ? HX_OK : fail(HX_ERR_HIP, "scale copy: %s", hipGetErrorString(e));
    }
  }
  uint64_t h[2] = {0, 0};
  if (!rc) {
    e = hipMemsetAsync(hdev, 0, 16, s);
    if (e != hipSuccess) rc = fail(HX_ERR_HIP, "hash clear: %s", hipGetErrorString(e));
  }
  if (!rc) rc = map_internal(launch_hash64(image, N * K * (int64_t)es, hdev, s), "hash");
  if (!rc && scale) rc = map_internal(launch_hash64(sc, N * 4, hdev + 1, s), "hash");
  if (!rc) {
    e = hipMemcpyAsync(h, hdev, 16, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) rc = fail(HX_ERR_HIP, "hash readback: %s", hipGetErrorString(e));
  }
  (void)hipFree(hdev);
  hdev = nullptr;
  if (rc) { cleanup(); return rc; }
  uint64_t key = h[0] ^ (h[1] * 0x9e3779b97f4a7c15ull) ^ ((uint64_t)K << 40) ^ ((uint64_t)N << 8) ^
                 (uint64_t)w_dtype ^ (scale ? 0x5ca1e5ull : 0);

  std::lock_guard<std::mutex> lk(g_mu);
  for (hx_weight* x : g_weights) {
    if (x->refcount > 0 && x->device == dev && x->hash == key && x->K == K && x->N == N &&
        x->dtype == w_dtype && (x->scale != nullptr) == (scale != nullptr)) {
      // A 64-bit key can collide: share the image only when the bytes
      // (image and scales) are equal, compared on the device.
      unsigned* cnt = nullptr;
      unsigned diff = 1;
      if (hipMalloc((void**)&cnt, sizeof(unsigned)) == hipSuccess) {
        bool ok = hipMemsetAsync(cnt, 0, sizeof(unsigned), s) == hipSuccess;
        ok = ok && launch_diff_bytes(image, x->image, N * K * (int64_t)es, cnt, s) == HXI_OK;
        if (ok && scale) ok = launch_diff_bytes(sc, x->scale, N * 4, cnt, s) == HXI_OK;
        ok = ok && hipMemcpyAsync(&diff, cnt, sizeof(unsigned), hipMemcpyDeviceToHost, s) == hipSuccess &&
             hipStreamSynchronize(s) == hipSuccess;
        (void)hipFree(cnt);
        if (!ok) {
          cleanup();
          return fail(HX_ERR_HIP, "hx_weight_register: content comparison failed");
        }
      }
      if (diff != 0) continue;  // same key, different content: a registration of its own
      ++x->refcount;
      cleanup();
      *out = x;
      return HX_OK;
    }
  }
  // the decode GEMV's image: every wave load one contiguous KiB (the [N][K]
  // image read in place gives sixteen 64-byte runs per load, about 1.4x
  // slower to stream)
  void* packed = nullptr;
  {
    const bool i8 = w_dtype == HX_I8;
    if (hipMalloc(&packed, (size_t)(i8 ? gemv_packed_bytes(N, K) : gemv_packed16_bytes(N, K))) != hipSuccess) {
      cleanup();
      return fail(HX_ERR_NOMEM, "packed weight image");
    }
    rc = map_internal(i8 ? launch_gemv_pack((const int8_t*)image, K, N, K, (int8_t*)packed, s)
                         : launch_gemv_pack16((const uint16_t*)image, K, N, K, (uint16_t*)packed, s),
                      "gemv pack");
    hipError_t se = hipStreamSynchronize(s);
    if (rc || se != hipSuccess) {
      (void)hipFree(packed);
      cleanup();
      return rc ? rc : fail(HX_ERR_HIP, "gemv pack: %s", hipGetErrorString(se));
    }
  }
  hx_weight* x = new hx_weight{dev, K, N, w_dtype, image, packed, sc, key, 1, 0};
  g_weights.insert(x);
  *out = x;
  return HX_OK;
}

extern "C" int hx_weight_release(hx_weight_t w) {
  free_deferred();
  {
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_weights.count(w) || w->refcount <= 0) return fail(HX_ERR_HANDLE, "hx_weight_release: unknown handle");
    if (--w->refcount > 0 || w->inuse > 0) return HX_OK;  // a running call frees it when it returns
    g_weights.erase(w);
  }
  weight_free(w);
  return HX_OK;
}

extern "C" int hx_weight_info(hx_weight_t w, int64_t* k, int64_t* n, int* dtype, uint64_t* content_hash,
                              int* refcount) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_weights.count(w) || w->refcount <= 0) return fail(HX_ERR_HANDLE, "hx_weight_info: unknown handle");
  if (k) *k = w->K;
  if (n) *n = w->N;
  if (dtype) *dtype = w->dtype;
  if (content_hash) *content_hash = w->hash;
  if (refcount) *refcount = w->refcount;
  return HX_OK;
}

// Whether a registered int8 weight's product with these activations runs
// the packed decode GEMV.  The packed GEMV reads activations as 8-element
// (16-byte) groups, with 32-bit buffer offsets into the activation rows and
// one workgroup's tiles.
// ffn: a product of the FFN block (gemv_rows4_i8).
static bool packed_gemv_takes(const View2& vx, const hx_weight* w, bool residual, int y_dt, bool ffn = false) {
  const int64_t M = vx.rows;
  const bool route = gemv_rows_route(M, w->N, true, true, w->K) || (ffn && gemv_rows4_i8(M, w->N, w->K, true));
  return w->dtype == HX_I8 && w->packed && route && !residual && y_dt == HX_F16 &&
         w->K % 8 == 0 && ((uintptr_t)vx.p & 15u) == 0 && (vx.ld * 2) % 16 == 0 &&
         M * vx.ld * 2 < ((int64_t)1 << 31) && (w->K + 63) / 64 * 4 * 1024 < ((int64_t)1 << 31);
}

// gate (int8 packed GEMV only, see packed_gemv_takes): the output becomes
// RNE(silu(gate) * RNE(x . W * s)), the SwiGLU gate fused into the epilogue.
static int matmul_resident_impl(const View2& vx, hx_weight* w, const View2* vr, int r_dt,
                                const View2& vy, int y_dt, hipStream_t s, const char* entry,
                                const PartialsTarget& pt = PartialsTarget{}, const View2* gate = nullptr,
                                bool ffn = false) {
  const int x_dt = w->dtype == HX_BF16 ? HX_BF16 : HX_F16;
  const int64_t M = vx.rows;
  if (M == 0) return HX_OK;
  if (gate && !packed_gemv_takes(vx, w, vr != nullptr, y_dt, ffn))
    return fail(HX_ERR_ARG, "%s: fused gate needs the packed decode GEMV", entry);
  if (packed_gemv_takes(vx, w, vr != nullptr, y_dt, ffn)) {
    GemvArgs v{};
    v.x = vx.p; v.ldx = vx.ld; v.w = nullptr; v.ldw = 0;
    v.scale = w->scale; v.y = vy.p; v.ldy = vy.ld; v.M = M; v.N = w->N; v.K = w->K;
    if (gate) { v.gate = (const uint16_t*)gate->p; v.ldg = gate->ld; }
    bool pin = false;
    const int cfg = resolve_gemv(HX_OP_GEMV_W8, M, w->N, w->K, &pin);
    if (pt.fixed) {
      // a K-split config's partials and counters come from the caller's
      // fixed scratch (the launcher would otherwise take the stream's own)
      const size_t need = gemv_split_bytes(cfg, M, w->N);
      if (need > pt.cap || (need && (!pt.buf || !pt.cnt)))
        return fail(HX_ERR_UNSUPPORTED, "%s: the decode GEMV's K split needs %zu bytes of scratch, %zu reserved",
                    entry, need, pt.cap);
      v.part = pt.buf; v.cnt = pt.cnt;
    }
    note_plan(PlanCtx{entry, "resident-packed", x_dt, w->dtype}, M, w->N, w->K, HX_F16, "gemv-packed",
              gemv_packed_config(cfg)->name, pin ? "pinned" : "default", M <= 16 ? "min-rows" : "few-rows");
    return map_internal(launch_gemv_packed(cfg, v, (const int8_t*)w->packed, s), "gemv_packed");
  }
  // f16 / bf16: the packed image (the [N][K] image read in place when the
  // packed path refuses the call)
  if (w->dtype != HX_I8 && gemv_rows_route(M, w->N, w->packed != nullptr, false, w->K) && !vr && y_dt == x_dt) {
    GemvArgs v{};
    v.x = vx.p; v.ldx = vx.ld; v.w = nullptr; v.ldw = 0;
    v.scale = w->scale; v.y = vy.p; v.ldy = vy.ld; v.M = M; v.N = w->N; v.K = w->K;
    // the packed image: activations as 16-byte groups, 32-bit offsets into
    // the activation rows and one workgroup's tiles (at most four)
    if (w->packed && !gemv_hw_refusal(w->dtype, v, w->image, w->K) && (w->K + 31) / 32 * 4 * 1024 < ((int64_t)1 << 31)) {
      const int op = w->dtype == HX_BF16 ? HX_OP_GEMV_BF16 : HX_OP_GEMV_F16;
      bool pin = false;
      const int cfg = resolve_gemv(op, M, w->N, w->K, &pin);
      note_plan(PlanCtx{entry, "resident-packed", x_dt, w->dtype}, M, w->N, w->K, x_dt, "gemv-packed",
                gemv_packed_config(cfg)->name, pin ? "pinned" : "default", M <= 16 ? "min-rows" : "few-rows");
      return map_internal(launch_gemv_packed16(cfg, w->dtype, v, w->packed, s), "gemv_packed");
    }
    if (!gemv_hw_refusal(w->dtype, v, w->image, w->K)) return run_gemv_hw(v, w->dtype, w->image, w->K, s,
                                                                PlanCtx{entry, "resident-image", x_dt, w->dtype});
  }
  GemmArgs g{};
  g.a = vx.p; g.lda = vx.ld;
  g.b = w->image; g.ldb = w->K;
  g.c = vy.p; g.ldc = vy.ld;
  g.M = M; g.N = w->N; g.K = w->K;
  g.out_dtype = y_dt;
  g.col_scale = w->scale;
  if (vr) { g.res = vr->p; g.ldr = vr->ld; g.res_dtype = r_dt; }
  const int op = w->dtype == HX_I8 ? HX_OP_MATMUL_W8 : w->dtype == HX_F16 ? HX_OP_MATMUL_F16 : HX_OP_MATMUL_BF16;
  return run_gemm(op, g, s, PlanCtx{entry, "resident-image", x_dt, w->dtype}, pt);
}

extern "C" int hx_matmul_resident(const hx_memref2d* x, int x_dtype, hx_weight_t wt,
                                  const hx_memref2d* residual, int residual_dtype, hx_memref2d* y,
                                  int y_dtype, hx_stream_t stream) {
  WeightUse use(wt);
  hx_weight* w = use.get();
  if (!w) return fail(HX_ERR_HANDLE, "hx_matmul_resident: unknown weight handle");
  const int want_x = w->dtype == HX_BF16 ? HX_BF16 : HX_F16;
  if (x_dtype != want_x)
    return fail(HX_ERR_DTYPE, "hx_matmul_resident: x is %s, weight %s needs %s", dt_name(x_dtype),
                dt_name(w->dtype), dt_name(want_x));
  if (y_dtype != HX_F16 && y_dtype != HX_BF16 && y_dtype != HX_F32)
    return fail(HX_ERR_DTYPE, "hx_matmul_resident: y dtype %s", dt_name(y_dtype));
  int rc, dev;
  if ((rc = current_device(&dev))) return rc;
  if (dev != w->device) return fail(HX_ERR_HANDLE, "hx_matmul_resident: weight lives on device %d", w->device);
  View2 vx, vy, vr;
  if ((rc = view2(x, x_dtype, "x", &vx)) || (rc = view2(y, y_dtype, "y", &vy))) return rc;
  if (vx.cols != w->K) return fail(HX_ERR_SHAPE, "hx_matmul_resident: x has K=%lld, weight K=%lld", (long long)vx.cols, (long long)w->K);
  if (vy.rows != vx.rows || vy.cols != w->N) return fail(HX_ERR_SHAPE, "hx_matmul_resident: y shape");
  if (residual) {
    if (residual_dtype != HX_F16 && residual_dtype != HX_BF16 && residual_dtype != HX_F32)
      return fail(HX_ERR_DTYPE, "hx_matmul_resident: residual dtype");
    if ((rc = view2(residual, residual_dtype, "residual", &vr))) return rc;
    if (vr.rows != vx.rows || vr.cols != w->N) return fail(HX_ERR_SHAPE, "hx_matmul_resident: residual shape");
  }
  return matmul_resident_impl(vx, w, residual ? &vr : nullptr, residual_dtype, vy, y_dtype,
                              (hipStream_t)stream, "hx_matmul_resident");
}

// The FFN block.  `fixed` (may be null) is caller-supplied device memory of
// fixed->cap bytes that holds every intermediate and K-split partial; then
// the call allocates nothing and refuses shapes that do not fit.  Without
// it the intermediates live in the stream's workspace.
int hx::swiglu_ffn_impl(const hx_memref2d* x, const hx_memref1d* gamma, float eps, hx_weight_t w_gate,
                        hx_weight_t w_up, hx_weight_t w_down, hx_memref2d* y, hx_stream_t stream,
                        const FixedScratch* fixed, const char* entry) {
  hipStream_t s = (hipStream_t)stream;
  WeightUse ug(w_gate, !fixed), uu(w_up, !fixed), ud(w_down, !fixed);
  hx_weight *wg = ug.get(), *wu = uu.get(), *wd = ud.get();
  if (!wg || !wu || !wd) return fail(HX_ERR_HANDLE, "%s: unknown weight handle", entry);
  if (wg->dtype != HX_I8 || wu->dtype != HX_I8 || wd->dtype != HX_I8)
    return fail(HX_ERR_DTYPE, "%s: int8 weights expected", entry);
  int rc, dev;
  if ((rc = current_device(&dev))) return rc;
  if (wg->device != dev || wu->device != dev || wd->device != dev)
    return fail(HX_ERR_HANDLE, "%s: weights live on another device", entry);
  View2 vx, vy;
  View1 vg{};
  if ((rc = view2(x, HX_F16, "x", &vx)) || (rc = view2(y, HX_F16, "y", &vy))) return rc;
  const int64_t T = vx.rows, H = vx.cols, I = wg->N;
  if (wg->K != H || wu->K != H || wu->N != I || wd->K != I || wd->N != H)
    return fail(HX_ERR_SHAPE, "%s: weights [%lld,%lld] [%lld,%lld] [%lld,%lld] vs hidden %lld", entry,
                (long long)wg->K, (long long)wg->N, (long long)wu->K, (long long)wu->N, (long long)wd->K,
                (long long)wd->N, (long long)H);
  if (vy.rows != T || vy.cols != H) return fail(HX_ERR_SHAPE, "%s: y shape", entry);
  if (gamma && (rc = view1(gamma, HX_F16, "gamma", H, &vg))) return rc;
  if (T == 0) return HX_OK;

  // up to 32 tokens: the decode GEMVs and their row blocks (H = 4096,
  // I = 11008, T = 17 / 24 / 32: 61.1 / 63.8 / 69.2 us against 76.0 / 78.4 /
  // 82.0 with the fused gate/up GEMM); up to 64 where all three products
  // take the packed GEMV's four row blocks (gemv_rows4_i8; H = 4096,
  // I = 11008, T = 33 / 48 / 64: 60.2 / 69.9 / 80.3 us against 84.6 / 86.0
  // / 87.1 through the GEMMs); beyond, the fused gate/up GEMM, whose down
  // projection still takes the row blocks where they win
  const bool skinny = T <= kGemvRowsMaxM ||
                      (T <= kGemvRowsMaxMI8 && packed_gemv_takes(View2{nullptr, T, H, H}, wg, false, HX_F16, true) &&
                       packed_gemv_takes(View2{nullptr, T, H, H}, wu, false, HX_F16, true) &&
                       packed_gemv_takes(View2{nullptr, T, I, I}, wd, false, HX_F16, true));
  Carver cv;
  const size_t off_h = cv.take((size_t)T * H * 2);
  const size_t off_a = cv.take((size_t)T * I * 2);
  // decode path: the up projection's epilogue applies the gate (silu(g)
  // u, as the silu_mul kernel would) when it runs the packed GEMV, so u
  // never leaves the kernel (the workspace's activations are 256-byte
  // aligned with rows of H halves)
  const bool fuse_gate = skinny && packed_gemv_takes(View2{nullptr, T, H, H}, wu, false, HX_F16, true);
  const size_t off_g = skinny ? cv.take((size_t)T * I * 2) : 0;
  const size_t off_u = skinny && !fuse_gate ? cv.take((size_t)T * I * 2) : 0;
  char* ws;
  PartialsTarget pt;
  if (fixed) {
    // the down projection's K-split partials (if its config splits) go in
    // the same scratch, after the intermediates
    ws = fixed->base;
    size_t part = 0;
    if (!skinny && packed_gemv_takes(View2{nullptr, T, I, I}, wd, false, HX_F16)) {
      // the down projection takes the packed GEMV's row blocks
      part = gemv_split_bytes(resolve_gemv(HX_OP_GEMV_W8, T, H, I), T, H);
    } else if (!skinny) {
      GemmArgs d{};
      d.a = ws + off_a; d.lda = I;
      d.b = wd->image; d.ldb = I;
      d.c = vy.p; d.ldc = vy.ld;
      d.M = T; d.N = H; d.K = I;
      d.out_dtype = HX_F16;
      d.col_scale = wd->scale;
      part = gemm_partials_needed(HX_OP_MATMUL_W8, d);
    } else {
      // the decode GEMVs' K-split partials (one region, the largest need of
      // the three products, which run one after another)
      part = std::max(gemv_split_bytes(resolve_gemv(HX_OP_GEMV_W8, T, I, H), T, I),
                      gemv_split_bytes(resolve_gemv(HX_OP_GEMV_W8, T, H, I), T, H));
    }
    const size_t off_p = part ? cv.take(part) : 0;
    if (cv.used > fixed->cap)
      return fail(HX_ERR_UNSUPPORTED, "%s: %lld tokens need %zu bytes of scratch; the fixed scratch holds %zu",
                  entry, (long long)T, cv.used, fixed->cap);
    pt.fixed = true;
    pt.buf = part ? reinterpret_cast<float*>(ws + off_p) : nullptr;
    pt.cap = part;
    pt.cnt = fixed->cnt;
  } else if ((rc = ws_get(s, cv.used, &ws))) {
    return rc;
  }
  char* h = ws + off_h;
  char* act = ws + off_a;
  rc = map_internal(launch_rmsnorm(HX_F16, vx.p, vx.ld, gamma ? vg.p : nullptr, eps, h, H, T, H, s), "rmsnorm");
  if (rc) return rc;
  View2 vh{h, T, H, H}, va{act, T, I, I};
  if (skinny) {
    View2 vgo{ws + off_g, T, I, I};
    if ((rc = matmul_resident_impl(vh, wg, nullptr, 0, vgo, HX_F16, s, entry, pt, nullptr, true))) return rc;
    if (fuse_gate) {
      if ((rc = matmul_resident_impl(vh, wu, nullptr, 0, va, HX_F16, s, entry, pt, &vgo, true))) return rc;
    } else {
      View2 vuo{ws + off_u, T, I, I};
      if ((rc = matmul_resident_impl(vh, wu, nullptr, 0, vuo, HX_F16, s, entry, pt, nullptr, true))) return rc;
      rc = map_internal(launch_silu_mul_f16(vgo.p, I, vuo.p, I, act, I, T, I, s), "silu_mul");
      if (rc) return rc;
    }
  } else {
    GemmArgs g{};
    g.a = h; g.lda = H;
    g.b = wg->image; g.b2 = wu->image; g.ldb = H;
    g.c = act; g.ldc = I;
    g.M = T; g.N = I; g.K = H;
    g.out_dtype = HX_F16;
    g.col_scale = wg->scale; g.col_scale2 = wu->scale;
    if ((rc = run_gemm(HX_OP_SWIGLU_W8, g, s, PlanCtx{entry, "resident-image", HX_F16, HX_I8}, pt))) return rc;
  }
  return matmul_resident_impl(va, wd, nullptr, 0, vy, HX_F16, s, entry, pt, nullptr, skinny);
}

extern "C" int hx_swiglu_ffn(const hx_memref2d* x, const hx_memref1d* gamma, float eps, hx_weight_t w_gate,
                             hx_weight_t w_up, hx_weight_t w_down, hx_memref2d* y, hx_stream_t stream) {
  return swiglu_ffn_impl(x, gamma, eps, w_gate, w_up, w_down, y, stream, nullptr, "hx_swiglu_ffn");
}

// ---------------------------------------------------------------------------
// Configurations
// ---------------------------------------------------------------------------
extern "C" int hx_config_count(int op) {
  std::vector<int> idx = family_indices(op);
  if (idx.empty()) return fail(HX_ERR_ARG, "hx_config_count: unknown op %d", op);
  return (int)idx.size();
}

extern "C" int hx_config_get(int op, int index, hx_kernel_config* out) {
  if (!out) return fail(HX_ERR_ARG, "hx_config_get: null out");
  std::vector<int> idx = family_indices(op);
  if (idx.empty()) return fail(HX_ERR_ARG, "hx_config_get: unknown op %d", op);
  if (index < 0 || index >= (int)idx.size()) return fail(HX_ERR_ARG, "hx_config_get: index %d", index);
  memset(out, 0, sizeof(*out));
  out->op = op;
  out->index = index;
  if (row_family(op)) {
    // lds_bytes: the two alternating exchange buffers of 2 x 4 floats
    out->col_tiles = row_config_per_cu(index);
    out->waves_m = out->col_tiles ? 4 : 0;
    out->lds_bytes = out->col_tiles ? 64 : 32;
    snprintf(out->name, sizeof(out->name), "%s", row_config_name(index));
    return HX_OK;
  }
  if (gemv_op(op)) {
    const GemvConfig* c = gemv_packed_config(idx[index]);
    // bm: activation rows one launch covers (16-row blocks); lds_bytes: the
    // cross-wave reduction buffer (reused per row block) plus, for configs
    // that stage the activation rows in LDS, the 64 KiB staging limit
    out->bm = 16 * c->mb; out->bn = 16 * c->ct; out->bk = op == HX_OP_GEMV_W8 ? 64 : 32;
    out->waves_m = c->kw; out->waves_n = 1;
    out->lds_stages = 0; out->split_k = c->split; out->col_tiles = c->ct;
    out->lds_bytes = c->kw * c->ct * 64 * 4 * 4 + (c->xl ? 65536 : 0);
    snprintf(out->name, sizeof(out->name), "gemv_%s", c->name);
    return HX_OK;
  }
  int mode, epi;
  op_gemm(op, &mode, &epi);
  const GemmConfig* c = gemm_config(mode, idx[index]);
  // bk: K elements per stage (sb bytes of A per row); brow: bytes of B per
  // row in one stage (the W8 weights are int8 beside f16 activations)
  const int bk = mode == GM_I8 ? c->sb : c->sb / 2;
  const int brow = mode == GM_W8 ? c->sb / 2 : c->sb;
  out->bm = c->bm; out->bn = c->bn; out->bk = bk;
  out->waves_m = c->wm; out->waves_n = c->wn;
  out->lds_stages = c->stages; out->split_k = c->ksplit > 1 ? c->ksplit : 1; out->col_tiles = 0;
  out->lds_bytes = c->stages * (c->bm * c->sb + (epi == GE_SWIGLU ? 2 : 1) * c->bn * brow);
  snprintf(out->name, sizeof(out->name), "%s", c->name);
  return HX_OK;
}

extern "C" int hx_config_select(int op, int64_t m, int64_t n, int64_t k, int index) {
  std::vector<int> idx = family_indices(op);
  if (idx.empty()) return fail(HX_ERR_ARG, "hx_config_select: unknown op %d", op);
  if (index < -1 || index >= (int)idx.size()) return fail(HX_ERR_ARG, "hx_config_select: index %d", index);
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_tuple(dev, op, m, n, k);
  if (index < 0) g_pins.erase(key);
  else g_pins[key] = index;
  return HX_OK;
}

static const char* config_name(int op, int index) {
  std::vector<int> idx = family_indices(op);
  if (index < 0 || index >= (int)idx.size()) return nullptr;
  if (row_family(op)) return row_config_name(index);
  if (gemv_op(op)) return gemv_packed_config(idx[index])->name;
  int mode, epi;
  op_gemm(op, &mode, &epi);
  return gemm_config(mode, idx[index])->name;
}

extern "C" int hx_config_pins_save(char* buf, size_t cap, size_t* needed) {
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  std::string out = "hx-pins/v2 " HX_BUILD_ID "\n";
  std::vector<std::pair<int, double>> canaries = canary_references(dev);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (const auto& kv : g_pins) {
      if (std::get<0>(kv.first) != dev) continue;
      const int op = std::get<1>(kv.first);
      char line[192];
      snprintf(line, sizeof(line), "pin %d %lld %lld %lld %d %s\n", op, (long long)std::get<2>(kv.first),
               (long long)std::get<3>(kv.first), (long long)std::get<4>(kv.first), kv.second,
               config_name(op, kv.second));
      out += line;
    }
  }
  for (const auto& c : canaries) {
    char line[96];
    snprintf(line, sizeof(line), "canary %d %.6g\n", c.first, c.second);
    out += line;
  }
  if (needed) *needed = out.size() + 1;
  if (!buf || cap < out.size() + 1)
    return fail(HX_ERR_ARG, "hx_config_pins_save: buffer of %zu bytes, %zu needed", cap, out.size() + 1);
  memcpy(buf, out.c_str(), out.size() + 1);
  return HX_OK;
}

extern "C" int hx_config_pins_load(const char* text) {
  if (!text) return fail(HX_ERR_ARG, "hx_config_pins_load: null text");
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  const std::string header = "hx-pins/v2 " HX_BUILD_ID;
  const char* nl = strchr(text, '\n');
  const std::string first = nl ? std::string(text, nl - text) : std::string(text);
  if (first != header)
    return fail(HX_ERR_ARG, "hx_config_pins_load: pins are from '%s', this library is '%s'", first.c_str(),
                header.c_str());
  // parse everything before applying anything
  std::vector<std::pair<std::tuple<int, int, int64_t, int64_t, int64_t>, int>> pins;
  std::vector<std::pair<int, double>> canaries;
  for (const char* line = nl ? nl + 1 : nullptr; line && *line;) {
    const char* end = strchr(line, '\n');
    const std::string l = end ? std::string(line, end - line) : std::string(line);
    line = end ? end + 1 : nullptr;
    if (l.empty()) continue;
    int op, index;
    long long m, n, k;
    char name[64];
    double q50;
    if (sscanf(l.c_str(), "pin %d %lld %lld %lld %d %63s", &op, &m, &n, &k, &index, name) == 6) {
      const char* have = config_name(op, index);
      if (!have || strcmp(have, name) != 0)
        return fail(HX_ERR_ARG, "hx_config_pins_load: op %d index %d is not config '%s'", op, index, name);
      pins.emplace_back(std::make_tuple(dev, op, (int64_t)m, (int64_t)n, (int64_t)k), index);
    } else if (sscanf(l.c_str(), "canary %d %lf", &op, &q50) == 2) {
      if (family_indices(op).empty() || !(q50 > 0.0) || !std::isfinite(q50))
        return fail(HX_ERR_ARG, "hx_config_pins_load: bad canary line '%s'", l.c_str());
      canaries.emplace_back(op, q50);
    } else {
      return fail(HX_ERR_ARG, "hx_config_pins_load: malformed line '%s'", l.c_str());
    }
  }
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (const auto& p : pins) g_pins[p.first] = p.second;
  }
  for (const auto& c : canaries) canary_reference_set(dev, c.first, c.second);
  return HX_OK;
}

extern "C" int hx_config_lookup(int op, int64_t m, int64_t n, int64_t k, int* index) {
  if (!index) return fail(HX_ERR_ARG, "hx_config_lookup: null out");
  std::vector<int> idx = family_indices(op);
  if (idx.empty()) return fail(HX_ERR_ARG, "hx_config_lookup: unknown op %d", op);
  int dev;
  int rc = current_device(&dev);
  if (rc) return rc;
  if (row_family(op)) {
    *index = resolve_row(op, m, n, (int)k);
    return HX_OK;
  }
  if (gemv_op(op)) {
    *index = resolve_gemv(op, m, n, k);
    return HX_OK;
  }
  const int t = resolve_gemm(op, m, n, k);
  *index = -1;
  for (size_t i = 0; i < idx.size(); ++i)
    if (idx[i] == t) *index = (int)i;
  return HX_OK;
}
