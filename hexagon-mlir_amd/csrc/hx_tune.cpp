// hx_tune.cpp -- the native autotuner: hx_tune times every compiled
// configuration of a kernel family at one shape on the caller's stream and
// picks (and optionally pins) a champion; hx_tune_decide is its decision
// rule alone, with no device work.
//
// What it replaces: the tile search of hexagon-mlir's host-side tuner
// (QHB/backend/hmx_search.py), i.e. candidate enumeration with legality
// (enumerate_tile_configs / tile_verdict, :246-332), timing with a per-config
// failure rule (hexagon_bench, :1109-1156; calibration_iters, :1159-1177), the
// noise-aware win margin (quantile_spread_cv / champion_gate, :1254-1289) and
// a per-round health probe (the canary, :1292-1368).
//
// The protocol constants are the reference's: three repetitions, quantiles
// (0.5, 0.2, 0.8), launches per repetition clamp(budget / one launch, 5,
// 1000), a failed or unverified configuration scores infinity, and a
// challenger must beat the default by more than max(3 CV, 15%).  The rest is
// this library's own design:
//   * candidates are the compiled configurations of a family (hx_config_get),
//     each run on synthetic seeded operands the tuner allocates for the
//     round (weights of bandwidth-bound families are rotated over enough
//     copies to exceed the 256 MB MALL, so HBM is what gets timed);
//   * every configuration's first launch writes into a poisoned output that
//     is compared on the device with the generic kernel's result (bit-equal
//     for int8, within 1e-2 relative for floats): a wrong kernel costs one
//     launch and scores infinity;
//   * timing is one HIP event pair per repetition on the caller's stream;
//   * the decision is a single comparison -- the fastest timed configuration
//     against the untuned default (the control arm) -- so the result does not
//     depend on the order the candidates were timed in;
//   * the canary is the untuned default configuration on a fixed small shape
//     of the family, re-timed after the sweep; its median is judged against
//     the median of the family's last valid round (held per device, saved and
//     loaded with the pins).  A shift beyond the canary's own gate means the
//     device moved while the round ran, and the round pins nothing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "../../include/hx.h"
#include "hx_api_internal.hpp"
#include "hx_device.hpp"
#include "hx_internal.hpp"

using namespace hx;

namespace {

constexpr double kInf = std::numeric_limits<double>::infinity();
constexpr double kCvFactor = 3.0;     // gate = max(3 CV, 15%)
constexpr double kGateFloor = 0.15;

double quantile(std::vector<double> v, double q) {
  if (v.empty()) return kInf;
  std::sort(v.begin(), v.end());
  const double pos = (double)(v.size() - 1) * q;
  const size_t lo = (size_t)pos;
  const size_t hi = std::min(lo + 1, v.size() - 1);
  const double f = pos - (double)lo;
  return v[lo] * (1.0 - f) + v[hi] * f;
}

// (q80 - q20) / q50; 0 when any is not finite or the median is not positive
double spread(const hx_tune_entry& e) {
  if (!std::isfinite(e.q20_us) || !std::isfinite(e.q50_us) || !std::isfinite(e.q80_us) || e.q50_us <= 0.0)
    return 0.0;
  return std::max(0.0, (e.q80_us - e.q20_us) / e.q50_us);
}

double gate_of(double cv) { return std::max(kCvFactor * cv, kGateFloor); }

bool timed(const hx_tune_entry& e) { return e.status == HX_TUNE_TIMED && std::isfinite(e.q50_us); }

void set_reason(hx_tune_entry& e, const char* r) {
  snprintf(e.reason, sizeof(e.reason), "%s", r);
}

// Device memory of one round, freed on every exit path.
struct Arena {
  std::vector<void*> ptrs;
  ~Arena() {
    for (void* p : ptrs) (void)hipFree(p);
  }
  void* get(size_t bytes) {
    void* p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 256) != hipSuccess) return nullptr;
    ptrs.push_back(p);
    return p;
  }
};

size_t es_of(int dt) { return dt == DT_I8 ? 1 : (dt == DT_F16 || dt == DT_BF16) ? 2 : 4; }

int64_t pad_pow2(int64_t x) {
  int64_t p = 32;
  while (p < x) p <<= 1;
  return p;
}

// One family at one shape: synthetic operands, the reference result of the
// generic kernel, and a launcher per configuration.
class Probe {
 public:
  Probe(int op, int64_t m, int64_t n, int64_t k, uint64_t seed, hipStream_t s)
      : op_(op), m_(m), n_(n), k_(k), seed_(seed), s_(s) {}

  // Allocate and fill the operands; HX_OK or an HX_ERR_* (text set).
  int setup() {
    idx_ = family_indices(op_);
    if (idx_.empty()) return api_fail(HX_ERR_ARG, "hx_tune: unknown op %d", op_);
    if (m_ <= 0 || n_ <= 0 || k_ <= 0) return api_fail(HX_ERR_SHAPE, "hx_tune: empty shape");
    cnt_ = (unsigned*)ar_.get(sizeof(unsigned));
    if (!cnt_) return api_fail(HX_ERR_NOMEM, "hx_tune: counter");
    return gemv_op(op_) ? setup_gemv() : setup_gemm();
  }

  int count() const { return (int)idx_.size(); }

  // Null when family config i may run at this shape, else why not.
  const char* refusal(int i) const {
    if (!family_reason_.empty()) return family_reason_.c_str();
    const int t = idx_[i];
    if (gemv_op(op_)) {
      const GemvConfig* c = gemv_packed_config(t);
      if (m_ > 16 * c->mb) return "rows-exceed-blocks";
      if (!gemv_xl_fits(*c, m_, k_, wt_)) return "staging-limit";
      if (c->split > 1 && !gemv_split_takes(*c, m_, n_)) return "split-rows";
      if (16 * c->ct > std::max<int64_t>(16, pad_pow2(n_))) return "tile-exceeds-extent";
      return nullptr;
    }
    const GemmConfig* c = gemm_config(mode_, t);
    if (c->bm > std::max<int64_t>(64, pad_pow2(m_)) || c->bn > std::max<int64_t>(64, pad_pow2(n_)))
      return "tile-exceeds-extent";
    if (c->ksplit > 1 && (k_ / c->ksplit) * es_of(ea_dt_) < 256) return "split-too-short";
    // a stage ring deeper than K runs (its extra stages load zeros): it is
    // timed like any other config
    return nullptr;
  }

  // Launch family config i on weight copy `copy`.
  int launch(int i, int copy) {
    const int t = idx_[i];
    int rc;
    if (!gemv_op(op_)) {
      rc = launch_gemm(mode_, t, g_[copy], s_);
    } else if (op_ == HX_OP_GEMV_W8) {
      rc = launch_gemv_packed(t, v_[copy], (const int8_t*)w_[copy], s_);
    } else {
      rc = launch_gemv_packed16(t, wt_, v_[copy], w_[copy], s_);
    }
    if (rc != HXI_OK) return HX_ERR_UNSUPPORTED;
    return hipGetLastError() == hipSuccess ? HX_OK : HX_ERR_HIP;
  }

  // Poison the output, launch config i once on copy 0, and compare with the
  // reference: *ok = whether it matched.
  int run_verified(int i, bool* ok) {
    *ok = false;
    if (hipMemsetAsync(out_, 0xff, out_bytes_, s_) != hipSuccess) return HX_ERR_HIP;
    int rc = launch(i, 0);
    if (rc) return rc;
    if (hipMemsetAsync(cnt_, 0, sizeof(unsigned), s_) != hipSuccess) return HX_ERR_HIP;
    const int64_t elems = (int64_t)(out_bytes_ / es_of(out_dt_));
    rc = exact_ ? launch_diff_bytes(out_, ref_, (int64_t)out_bytes_, cnt_, s_)
                : launch_count_far(out_, ref_, elems, out_dt_, 1e-2f, 1e-2f, cnt_, s_);
    if (rc != HXI_OK) return HX_ERR_HIP;
    unsigned bad = 1;
    if (hipMemcpyAsync(&bad, cnt_, sizeof(unsigned), hipMemcpyDeviceToHost, s_) != hipSuccess ||
        hipStreamSynchronize(s_) != hipSuccess)
      return HX_ERR_HIP;
    *ok = bad == 0;
    return HX_OK;
  }

  // Mean device time (us) per launch of `iters` launches of config i,
  // rotating over the weight copies; HX_OK or an error.
  int time(int i, int iters, double* us) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return HX_ERR_HIP;
    if (hipEventCreate(&e1) != hipSuccess) {
      (void)hipEventDestroy(e0);
      return HX_ERR_HIP;
    }
    int rc = hipEventRecord(e0, s_) == hipSuccess ? HX_OK : HX_ERR_HIP;
    for (int it = 0; it < iters && !rc; ++it) rc = launch(i, it % copies_);
    if (!rc && hipEventRecord(e1, s_) != hipSuccess) rc = HX_ERR_HIP;
    float ms = 0.f;
    if (!rc && (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess))
      rc = HX_ERR_HIP;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (!rc) *us = 1000.0 * (double)ms / iters;
    return rc;
  }

 private:
  int fill(void* p, int64_t n, int dt, float lo, float hi, uint64_t salt) {
    return launch_fill_uniform(p, n, dt, lo, hi, seed_ * 1000003ull + salt, s_) == HXI_OK ? HX_OK
                                                                                        : HX_ERR_HIP;
  }

  // Weight copies: enough to exceed twice the 256 MB MALL for a
  // bandwidth-bound family, at most 16; one for the compute-bound GEMMs.
  int copies_for(size_t weight_bytes, bool streamed) const {
    if (!streamed) return 1;
    const size_t want = (size_t)600 << 20;
    size_t c = (want + weight_bytes - 1) / weight_bytes;
    return (int)std::max<size_t>(1, std::min<size_t>(c, 16));
  }

  int setup_gemm() {
    int epi;
    op_gemm(op_, &mode_, &epi);
    ea_dt_ = mode_ == GM_I8 ? DT_I8 : mode_ == GM_BF16 ? DT_BF16 : DT_F16;
    const int eb_dt = (mode_ == GM_I8 || mode_ == GM_W8) ? DT_I8 : ea_dt_;
    out_dt_ = mode_ == GM_BF16 ? DT_BF16 : DT_F16;
    exact_ = mode_ == GM_I8;
    const size_t ea = es_of(ea_dt_), eb = es_of(eb_dt);
    const bool swiglu = epi == GE_SWIGLU;
    // skinny M streams its weight: rotate copies as the GEMV does
    copies_ = copies_for((size_t)n_ * k_ * eb * (swiglu ? 2 : 1), m_ <= 64);
    void* a = ar_.get((size_t)m_ * k_ * ea);
    out_bytes_ = (size_t)m_ * n_ * es_of(out_dt_);
    out_ = ar_.get(out_bytes_);
    ref_ = ar_.get(out_bytes_);
    if (!a || !out_ || !ref_) return api_fail(HX_ERR_NOMEM, "hx_tune: operands of %lldx%lldx%lld",
                                              (long long)m_, (long long)n_, (long long)k_);
    const float lo = ea_dt_ == DT_I8 ? -127.f : -1.f, hi = -lo;
    if (fill(a, m_ * k_, ea_dt_, lo, hi, 1)) return api_fail(HX_ERR_HIP, "hx_tune: fill");
    // scales: the dequant range of the int8 GEMM, and per-channel scales
    // that keep the W8A16 outputs O(1)
    float* rs = nullptr;
    float* cs = nullptr;
    float* cs2 = nullptr;
    const float wlo = 0.5f / (127.f * sqrtf((float)k_ / 3.f)), whi = 3.f * wlo;
    if (mode_ == GM_I8) {
      rs = (float*)ar_.get((size_t)m_ * 4);
      cs = (float*)ar_.get((size_t)n_ * 4);
      if (!rs || !cs || fill(rs, m_, DT_F32, 0.001f, 0.02f, 2) || fill(cs, n_, DT_F32, 0.001f, 0.02f, 3))
        return api_fail(HX_ERR_NOMEM, "hx_tune: scales");
    } else if (mode_ == GM_W8) {
      cs = (float*)ar_.get((size_t)n_ * 4);
      if (!cs || fill(cs, n_, DT_F32, wlo, whi, 3)) return api_fail(HX_ERR_NOMEM, "hx_tune: scales");
      if (swiglu) {
        cs2 = (float*)ar_.get((size_t)n_ * 4);
        if (!cs2 || fill(cs2, n_, DT_F32, wlo, whi, 4)) return api_fail(HX_ERR_NOMEM, "hx_tune: scales");
      }
    }
    const float blo = eb_dt == DT_I8 ? -127.f : -1.f, bhi = -blo;
    size_t part = 0;
    for (int i = 0; i < count(); ++i) {
      GemmArgs t{};
      t.M = m_; t.N = n_; t.K = k_;
      part = std::max(part, gemm_part_bytes(mode_, idx_[i], t));
    }
    float* partials = nullptr;
    unsigned* split_cnt = nullptr;
    if (part) {
      // the split configs merge inside the kernel with per-tile counters
      // (zero here; every launch leaves them at zero), as the products run
      if (!(partials = (float*)ar_.get(part)) ||
          !(split_cnt = (unsigned*)ar_.get((size_t)kGemvSplitCounters * sizeof(unsigned))))
        return api_fail(HX_ERR_NOMEM, "hx_tune: partials");
      if (launch_fill_u32(split_cnt, kGemvSplitCounters, 0u, s_) != HXI_OK || hipGetLastError() != hipSuccess)
        return api_fail(HX_ERR_HIP, "hx_tune: clearing the split counters");
    }
    for (int c = 0; c < copies_; ++c) {
      void* b = ar_.get((size_t)n_ * k_ * eb);
      void* b2 = swiglu ? ar_.get((size_t)n_ * k_ * eb) : nullptr;
      if (!b || (swiglu && !b2)) return api_fail(HX_ERR_NOMEM, "hx_tune: weight copy %d", c);
      if (fill(b, n_ * k_, eb_dt, blo, bhi, 10 + 2 * c) || (b2 && fill(b2, n_ * k_, eb_dt, blo, bhi, 11 + 2 * c)))
        return api_fail(HX_ERR_HIP, "hx_tune: fill");
      GemmArgs g{};
      g.a = a; g.lda = k_;
      g.b = b; g.ldb = k_; g.b2 = b2;
      g.c = out_; g.ldc = n_;
      g.M = m_; g.N = n_; g.K = k_;
      g.out_dtype = out_dt_;
      g.row_scale = rs; g.col_scale = cs; g.col_scale2 = cs2;
      g.part = partials;
      g.cnt = split_cnt;
      g_.push_back(g);
    }
    if (const char* why = gemm_fast_refusal(mode_, g_[0])) family_reason_ = why;
    GemmArgs r = g_[0];
    r.c = ref_;
    if (launch_gemm_generic(mode_, r, s_) != HXI_OK || hipGetLastError() != hipSuccess)
      return api_fail(HX_ERR_HIP, "hx_tune: reference launch");
    return HX_OK;
  }

  int setup_gemv() {
    wt_ = op_ == HX_OP_GEMV_W8 ? DT_I8 : op_ == HX_OP_GEMV_BF16 ? DT_BF16 : DT_F16;
    const int xt = op_ == HX_OP_GEMV_BF16 ? DT_BF16 : DT_F16;
    out_dt_ = xt;
    exact_ = false;
    // the shapes the products run on this family (a registered weight's
    // packed image)
    if (m_ > kGemvMaxRows || !gemv_rows_route(m_, n_, true, op_ == HX_OP_GEMV_W8, k_)) family_reason_ = "family-shape";
    const int64_t mm = std::min<int64_t>(m_, kGemvMaxRows);
    const size_t eb = es_of(wt_);
    // every family times the registered weight's packed image, the form a
    // resident decode reads (a pin applies to an argument [N][K] weight
    // read in place as well)
    const size_t img = op_ == HX_OP_GEMV_W8 ? (size_t)gemv_packed_bytes(n_, k_) : (size_t)gemv_packed16_bytes(n_, k_);
    copies_ = copies_for(img, true);
    void* x = ar_.get((size_t)mm * k_ * 2);
    out_bytes_ = (size_t)mm * n_ * 2;
    out_ = ar_.get(out_bytes_);
    ref_ = ar_.get(out_bytes_);
    // [N][K] image of copy 0: the reference's operand and the source of
    // copy 0's packed image; copies >= 1 are generated into a scratch image
    // and packed from there
    void* w0 = ar_.get((size_t)n_ * k_ * eb);
    void* scratch = copies_ > 1 ? ar_.get((size_t)n_ * k_ * eb) : nullptr;
    if (!x || !out_ || !ref_ || !w0 || (copies_ > 1 && !scratch))
      return api_fail(HX_ERR_NOMEM, "hx_tune: operands");
    if (fill(x, mm * k_, xt, -1.f, 1.f, 1)) return api_fail(HX_ERR_HIP, "hx_tune: fill");
    float* sc = nullptr;
    if (wt_ == DT_I8) {
      sc = (float*)ar_.get((size_t)n_ * 4);
      if (!sc || fill(sc, n_, DT_F32, 0.001f, 0.02f, 3)) return api_fail(HX_ERR_NOMEM, "hx_tune: scales");
    }
    const float lo = wt_ == DT_I8 ? -127.f : -1.f, hi = -lo;
    ref_nk_ = w0;
    for (int c = 0; c < copies_; ++c) {
      void* nk = c == 0 ? w0 : scratch;
      if (fill(nk, n_ * k_, wt_, lo, hi, 10 + c)) return api_fail(HX_ERR_HIP, "hx_tune: fill");
      // the registered (resident) form the decode GEMV reads
      void* packed = ar_.get(img);
      if (!packed) return api_fail(HX_ERR_NOMEM, "hx_tune: packed copy %d", c);
      const int prc = wt_ == DT_I8 ? launch_gemv_pack((const int8_t*)nk, k_, n_, k_, (int8_t*)packed, s_)
                                   : launch_gemv_pack16((const uint16_t*)nk, k_, n_, k_, (uint16_t*)packed, s_);
      if (prc != HXI_OK) return api_fail(HX_ERR_HIP, "hx_tune: pack");
      w_.push_back(packed);
      GemvArgs v{};
      v.x = x; v.ldx = k_;
      v.scale = sc;
      v.y = out_; v.ldy = n_;
      v.M = mm; v.N = n_; v.K = k_;
      v_.push_back(v);
    }
    if (family_reason_.empty() && wt_ != DT_I8) {
      if (const char* why = gemv_hw_refusal(wt_, v_[0], w_[0], k_)) family_reason_ = why;
      else if ((k_ + 31) / 32 * 4 * 1024 >= ((int64_t)1 << 31)) family_reason_ = "offset-range";
    }
    if (family_reason_.empty() && wt_ == DT_I8 && k_ % 8 != 0) family_reason_ = "k-granularity";
    return reference_gemv();
  }

  int reference_gemv() {
    // the generic GEMM on copy 0's [N][K] weight
    GemmArgs r{};
    r.a = v_[0].x; r.lda = k_;
    r.b = ref_nk_; r.ldb = k_;
    r.c = ref_; r.ldc = n_;
    r.M = v_[0].M; r.N = n_; r.K = k_;
    r.out_dtype = out_dt_;
    r.col_scale = v_[0].scale;
    const int mode = wt_ == DT_I8 ? GM_W8 : wt_ == DT_BF16 ? GM_BF16 : GM_F16;
    if (!r.b) return api_fail(HX_ERR_ARG, "hx_tune: reference weight");
    if (launch_gemm_generic(mode, r, s_) != HXI_OK || hipGetLastError() != hipSuccess)
      return api_fail(HX_ERR_HIP, "hx_tune: reference launch");
    return HX_OK;
  }

 public:
  int op_;
  int64_t m_, n_, k_;
  uint64_t seed_;
  hipStream_t s_;
  Arena ar_;
  std::vector<int> idx_;
  std::string family_reason_;
  unsigned* cnt_ = nullptr;
  int mode_ = 0, ea_dt_ = DT_F16, wt_ = DT_F16, out_dt_ = DT_F16;
  bool exact_ = false;
  int copies_ = 1;
  void* out_ = nullptr;
  void* ref_ = nullptr;
  size_t out_bytes_ = 0;
  std::vector<GemmArgs> g_;
  std::vector<GemvArgs> v_;
  std::vector<const void*> w_;
  const void* ref_nk_ = nullptr;
};

}  // namespace

extern "C" int hx_tune_decide(const hx_tune_entry* entries, int n, int control_index, const hx_tune_entry* canary,
                              double canary_reference_us, hx_tune_report* out) {
  if (!out || (n > 0 && !entries) || n < 0) return api_fail(HX_ERR_ARG, "hx_tune_decide: null argument");
  // the fastest timed configuration (ties go to the lower index)
  int best = -1;
  for (int i = 0; i < n; ++i)
    if (timed(entries[i]) && (best < 0 || entries[i].q50_us < entries[best].q50_us)) best = i;
  out->best_index = best >= 0 ? entries[best].index : -1;
  out->best_q50_us = best >= 0 ? entries[best].q50_us : kInf;
  int ctrl = -1;
  for (int i = 0; i < n; ++i)
    if (entries[i].index == control_index) ctrl = i;
  out->control_index = control_index;
  out->control_q50_us = ctrl >= 0 && timed(entries[ctrl]) ? entries[ctrl].q50_us : kInf;
  if (best < 0) {
    // nothing ran: there is no champion
    out->champion_index = -1;
    out->margin = 0.0;
    out->gate = kGateFloor;
  } else if (ctrl < 0 || !timed(entries[ctrl])) {
    // no control measurement to defend: the fastest configuration is the
    // only evidence there is
    out->champion_index = entries[best].index;
    out->margin = 0.0;
    out->gate = gate_of(spread(entries[best]));
  } else {
    const hx_tune_entry& c = entries[ctrl];
    const hx_tune_entry& b = entries[best];
    out->margin = (c.q50_us - b.q50_us) / c.q50_us;
    out->gate = gate_of(std::max(spread(c), spread(b)));
    out->champion_index = out->margin > out->gate ? b.index : c.index;
  }
  // the canary
  out->canary_reference_us = canary_reference_us > 0.0 ? canary_reference_us : 0.0;
  out->canary_q50_us = canary && timed(*canary) ? canary->q50_us : kInf;
  out->canary_shift = 0.0;
  out->canary_gate = canary && timed(*canary) ? gate_of(spread(*canary)) : kGateFloor;
  if (!canary || !timed(*canary)) {
    out->canary_status = HX_CANARY_FAILED;
  } else if (!(canary_reference_us > 0.0) || !std::isfinite(canary_reference_us)) {
    out->canary_status = HX_CANARY_BASELINE;
  } else {
    out->canary_shift = (canary->q50_us - canary_reference_us) / canary_reference_us;
    out->canary_status = std::fabs(out->canary_shift) > out->canary_gate ? HX_CANARY_DRIFT : HX_CANARY_STEADY;
  }
  out->round_valid = out->canary_status == HX_CANARY_BASELINE || out->canary_status == HX_CANARY_STEADY;
  return HX_OK;
}

namespace {

// The canary probe of a family: its untuned default on a small fixed shape.
void canary_shape(int op, int64_t* m, int64_t* n, int64_t* k) {
  if (gemv_op(op)) {
    *m = 1; *n = 2048; *k = 2048;
  } else {
    *m = 256; *n = 256; *k = 256;
  }
}

struct Protocol {
  int reps, min_iters, max_iters;
  double budget_us;
};

// Time family config i of probe p with the protocol: warm-up + first-launch
// check, calibration, then reps repetitions.  Fills the entry's status and
// quantiles; *iters_out = launches per repetition used.
void measure(Probe& p, int i, const Protocol& pr, hx_tune_entry* e, int* iters_out) {
  e->q50_us = e->q20_us = e->q80_us = kInf;
  bool ok = false;
  if (p.run_verified(i, &ok) != HX_OK) {
    e->status = HX_TUNE_LAUNCH_FAILED;
    set_reason(*e, "launch-failed");
    (void)hipGetLastError();
    return;
  }
  if (!ok) {
    e->status = HX_TUNE_WRONG;
    set_reason(*e, "verify-failed");
    return;
  }
  double one = 0.0;
  if (p.time(i, 3, &one) != HX_OK || !(one > 0.0)) {
    e->status = HX_TUNE_LAUNCH_FAILED;
    set_reason(*e, "timing-failed");
    (void)hipGetLastError();
    return;
  }
  const double want = pr.budget_us / std::max(one, 1.0);
  const int iters = (int)std::max<double>(pr.min_iters, std::min<double>(pr.max_iters, want));
  std::vector<double> samples;
  for (int r = 0; r < pr.reps; ++r) {
    double us = 0.0;
    if (p.time(i, iters, &us) != HX_OK || !std::isfinite(us)) {
      e->status = HX_TUNE_LAUNCH_FAILED;
      set_reason(*e, "timing-failed");
      (void)hipGetLastError();
      return;
    }
    samples.push_back(us);
  }
  e->status = HX_TUNE_TIMED;
  e->q50_us = quantile(samples, 0.5);
  e->q20_us = quantile(samples, 0.2);
  e->q80_us = quantile(samples, 0.8);
  set_reason(*e, "timed");
  if (iters_out) *iters_out = iters;
}

}  // namespace

extern "C" int hx_tune(int op, int64_t m, int64_t n, int64_t k, const hx_tune_options* opt, hx_tune_report* out,
                       hx_stream_t stream) {
  if (!out) return api_fail(HX_ERR_ARG, "hx_tune: null report");
  memset(out, 0, sizeof(*out));
  out->op = op;
  out->m = m; out->n = n; out->k = k;
  out->champion_index = out->best_index = out->control_index = -1;
  hx_tune_options o{};
  if (opt) o = *opt;
  Protocol pr{o.reps > 0 ? o.reps : 3, o.min_iters > 0 ? o.min_iters : 5, o.max_iters > 0 ? o.max_iters : 1000,
              o.budget_us > 0.0 ? o.budget_us : 2.0e6};
  if (pr.max_iters < pr.min_iters) pr.max_iters = pr.min_iters;
  const uint64_t seed = o.seed ? o.seed : 0x5eed;
  hipStream_t s = (hipStream_t)stream;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return api_fail(HX_ERR_NODEVICE, "hx_tune: no device");
  if (family_indices(op).empty()) return api_fail(HX_ERR_ARG, "hx_tune: unknown op %d", op);
  if (row_family(op))
    return api_fail(HX_ERR_UNSUPPORTED, "hx_tune: row family %d is not tuned (pin it with hx_config_select)", op);
  if (family_indices(op).size() > HX_TUNE_MAX_ENTRIES)
    return api_fail(HX_ERR_UNSUPPORTED, "hx_tune: family %d has more than %d configs", op, HX_TUNE_MAX_ENTRIES);

  std::vector<hx_tune_entry> entries;
  {
    Probe p(op, m, n, k, seed, s);
    int rc = p.setup();
    if (rc) return rc;
    for (int i = 0; i < p.count(); ++i) {
      hx_tune_entry e{};
      e.index = i;
      e.q50_us = e.q20_us = e.q80_us = kInf;
      if (const char* why = p.refusal(i)) {
        e.status = HX_TUNE_REFUSED;
        set_reason(e, why);
      } else {
        int iters = 0;
        measure(p, i, pr, &e, &iters);
        if (iters > out->iters) out->iters = iters;
      }
      entries.push_back(e);
    }
  }  // the sweep's operands are freed before the canary runs

  // the canary: the family's untuned default on its fixed probe shape
  int64_t cm, cn, ck;
  canary_shape(op, &cm, &cn, &ck);
  out->canary_m = cm; out->canary_n = cn; out->canary_k = ck;
  hx_tune_entry canary{};
  canary.index = untuned_family_index(op, cm, cn, ck);
  canary.q50_us = canary.q20_us = canary.q80_us = kInf;
  out->canary_index = canary.index;
  {
    Probe p(op, cm, cn, ck, seed ^ 0xca4a41ull, s);
    if (canary.index >= 0 && p.setup() == HX_OK && !p.refusal(canary.index)) {
      measure(p, canary.index, pr, &canary, nullptr);
    } else {
      canary.status = HX_TUNE_LAUNCH_FAILED;
      set_reason(canary, "probe-unavailable");
    }
  }
  double ref = 0.0;
  if (o.canary_reference_us > 0.0) ref = o.canary_reference_us;
  else if (o.canary_reference_us == 0.0 && !canary_reference_get(dev, op, &ref)) ref = 0.0;
  else if (o.canary_reference_us < 0.0) ref = 0.0;

  const int control = untuned_family_index(op, m, n, k);
  hx_tune_decide(entries.data(), (int)entries.size(), control, &canary, ref, out);
  out->n_entries = (int)entries.size();
  for (size_t i = 0; i < entries.size(); ++i) out->entries[i] = entries[i];
  if (out->round_valid) canary_reference_set(dev, op, canary.q50_us);
  out->pinned = 0;
  if (out->round_valid && o.pin && out->champion_index >= 0) {
    int rc = hx_config_select(op, m, n, k, out->champion_index);
    if (rc) return rc;
    out->pinned = 1;
  }
  return HX_OK;
}
