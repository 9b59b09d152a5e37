// wrapper_driver.cpp -- a C++ caller of libhxmi with no Python and no torch:
// what the reference's generated kernel wrapper becomes when it routes its
// operators to the MI355X library (the launcher-emitted main() that builds
// MemRefDescriptors and calls the compiled kernel,
// hexagon_launcher_base.py:40-95; test/python/mlir/add_2d_kernel/
// wrapper.cpp:24-61).  It allocates with hipMalloc, fills operands from a
// seeded host generator, converts MLIR-style descriptors to the hx ones,
// calls the C ABI (matmul with residual, int8 GEMM with dequant, row ops,
// a registered weight through the decode GEMV, the native tuner, the pins
// text, an error path) and checks every result against the CPU oracle
// (oracle/hx_oracle.c, linked in as the checker).
//
// Test infrastructure: built by __graft_entry__.build() into
// tests/cpp/hx_wrapper_driver, run by tests/test_gpu_cpp_wrapper.py.
// Prints one "PASS <case>" / "FAIL <case> ..." line per case and
// "ALL PASS" when every case passed; exit status 0 only then.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "hx.h"

extern "C" {
// the CPU oracle (oracle/hx_oracle.c)
uint16_t hxo_f32_to_f16(float f);
float hxo_f16_to_f32(uint16_t h);
void hxo_gemm_i8_i32(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb, int b_trans, int32_t* C,
                     int64_t ldc, int64_t M, int64_t N, int64_t K);
void hxo_dequant_i32_f16(const int32_t* C, int64_t ldc, const float* sa, const float* sb, uint16_t* out,
                         int64_t ldo, int64_t M, int64_t N);
void hxo_matmul(const void* A, int a_dtype, int64_t lda, const void* B, int b_dtype, int64_t ldb, int b_trans,
                const float* scale_n, const void* R, int r_dtype, int64_t ldr, void* C, int c_dtype, int64_t ldc,
                int64_t M, int64_t N, int64_t K);
void hxo_softmax(const void* x, void* y, int dtype, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy);
void hxo_rmsnorm(const void* x, const void* gamma, float eps, void* y, int dtype, int64_t rows, int64_t cols,
                 int64_t ldx, int64_t ldy);
}

// MLIR's ranked memref descriptor (CRunnerUtils.h), the type the
// reference's wrapper holds.
template <class T, int N>
struct MemRefDescriptor {
  T* allocated;
  T* aligned;
  int64_t offset;
  int64_t sizes[N];
  int64_t strides[N];
};

template <class T>
static hx_memref2d to_hx(const MemRefDescriptor<T, 2>& d) {
  hx_memref2d m;
  m.allocated = (void*)d.allocated;
  m.aligned = (void*)d.aligned;
  m.offset = d.offset;
  for (int i = 0; i < 2; ++i) m.sizes[i] = d.sizes[i], m.strides[i] = d.strides[i];
  return m;
}
template <class T>
static hx_memref1d to_hx(const MemRefDescriptor<T, 1>& d) {
  hx_memref1d m;
  m.allocated = (void*)d.allocated;
  m.aligned = (void*)d.aligned;
  m.offset = d.offset;
  m.sizes[0] = d.sizes[0];
  m.strides[0] = d.strides[0];
  return m;
}

// ---- host-side helpers -----------------------------------------------------

static uint64_t g_state = 0x9e3779b97f4a7c15ull;
static uint64_t splitmix64() {
  uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static double unit() { return (double)(splitmix64() >> 11) * (1.0 / 9007199254740992.0); }
static float uniform(float lo, float hi) { return lo + (hi - lo) * (float)unit(); }
static float normal(float sd) {
  const double u1 = unit() + 1e-300, u2 = unit();
  return (float)(sd * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}

static bool hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::printf("FAIL hip %s: %s\n", what, hipGetErrorString(e));
    return false;
  }
  return true;
}

// A device buffer holding a copy of a host vector.
template <class T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  explicit DevBuf(const std::vector<T>& h) : n(h.size()) {
    hip_ok(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
    hip_ok(hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
  }
  explicit DevBuf(size_t count) : n(count) {
    hip_ok(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
    hip_ok(hipMemset(p, 0, n * sizeof(T)), "hipMemset");
  }
  ~DevBuf() { (void)hipFree(p); }
  std::vector<T> get() const {
    std::vector<T> h(n);
    hip_ok(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return h;
  }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
};

template <class T>
static MemRefDescriptor<T, 2> desc2(T* p, int64_t rows, int64_t cols, int64_t ld) {
  return MemRefDescriptor<T, 2>{p, p, 0, {rows, cols}, {ld, 1}};
}
template <class T>
static MemRefDescriptor<T, 1> desc1(T* p, int64_t n) {
  return MemRefDescriptor<T, 1>{p, p, 0, {n}, {1}};
}

static std::vector<uint16_t> f16_vec(size_t n, float (*gen)()) {
  std::vector<uint16_t> v(n);
  for (auto& x : v) x = hxo_f32_to_f16(gen());
  return v;
}

// Elementwise |got - want| <= atol + rtol |want| on f16 (or f32) data.
template <class T>
static bool close(const std::vector<T>& got, const std::vector<T>& want, float rtol, float atol,
                  const char* name) {
  size_t bad = 0, first = 0;
  double worst = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    float g, w;
    if constexpr (sizeof(T) == 2) g = hxo_f16_to_f32(got[i]), w = hxo_f16_to_f32(want[i]);
    else g = (float)got[i], w = (float)want[i];
    const double err = std::fabs((double)g - (double)w);
    if (!(err <= atol + rtol * std::fabs((double)w))) {
      if (bad++ == 0) first = i;
      if (err > worst) worst = err;
    }
  }
  if (bad) {
    std::printf("FAIL %s: %zu of %zu elements outside rtol %g atol %g (first index %zu, worst %g)\n", name, bad,
                got.size(), rtol, atol, first, worst);
    return false;
  }
  return true;
}

static int g_failed = 0;
static void report(bool ok, const char* name) {
  if (ok) std::printf("PASS %s\n", name);
  else ++g_failed;
  std::fflush(stdout);
}
static bool rc_ok(int rc, const char* what) {
  if (rc != HX_OK) {
    std::printf("FAIL %s returned %d: %s\n", what, rc, hx_last_error());
    return false;
  }
  return true;
}

// ---- cases -------------------------------------------------------------------

// C1: fp16 C = A.B + C_res with an f32 residual (the matmul-with-init case,
// MatmulToHmxPass.cpp:100-121), B in linalg [K][N].
static void case_matmul_residual(hipStream_t s) {
  const int64_t M = 256, N = 256, K = 256;
  auto a = f16_vec(M * K, [] { return uniform(-1.f, 1.f); });
  auto b = f16_vec(K * N, [] { return uniform(-1.f, 1.f); });
  std::vector<float> r(M * N);
  for (auto& x : r) x = uniform(-1.f, 1.f);
  DevBuf<uint16_t> da(a), db(b);
  DevBuf<float> dc(r);
  auto A = desc2(da.p, M, K, K);
  auto B = desc2(db.p, K, N, N);
  auto C = desc2(dc.p, M, N, N);
  hx_memref2d ma = to_hx(A), mb = to_hx(B), mc = to_hx(C);
  bool ok = rc_ok(hx_matmul(&ma, HX_F16, &mb, HX_F16, HX_LAYOUT_KN, nullptr, 0, &mc, HX_F32, &mc, HX_F32, s),
                  "hx_matmul");
  ok = ok && hip_ok(hipStreamSynchronize(s), "sync");
  if (ok) {
    std::vector<float> want(M * N);
    hxo_matmul(a.data(), HX_F16, K, b.data(), HX_F16, N, 0, nullptr, r.data(), HX_F32, N, want.data(), HX_F32,
               N, M, N, K);
    ok = close(dc.get(), want, 1e-2f, 1e-3f, "matmul_f16_f32_residual");
  }
  report(ok, "matmul_f16_f32_residual_256");
}

// C2-shaped int8 GEMM (smaller): exact int32, and the fp16 dequant bit-exact.
static void case_gemm_i8(hipStream_t s) {
  const int64_t M = 512, N = 384, K = 640;
  std::vector<int8_t> a(M * K), bt(N * K);
  for (auto& x : a) x = (int8_t)((int)(splitmix64() % 255) - 127);
  for (auto& x : bt) x = (int8_t)((int)(splitmix64() % 255) - 127);
  std::vector<float> sa(M), sb(N);
  for (auto& x : sa) x = uniform(0.001f, 0.02f);
  for (auto& x : sb) x = uniform(0.001f, 0.02f);
  DevBuf<int8_t> da(a), db(bt);
  DevBuf<float> dsa(sa), dsb(sb);
  DevBuf<int32_t> d32(M * N);
  DevBuf<uint16_t> d16(M * N);
  hx_memref2d ma = to_hx(desc2(da.p, M, K, K)), mb = to_hx(desc2(db.p, N, K, K));
  hx_memref2d m32 = to_hx(desc2(d32.p, M, N, N)), m16 = to_hx(desc2(d16.p, M, N, N));
  hx_memref1d msa = to_hx(desc1(dsa.p, M)), msb = to_hx(desc1(dsb.p, N));
  bool ok = rc_ok(hx_gemm_i8(&ma, &mb, HX_LAYOUT_NK, nullptr, nullptr, &m32, HX_I32, s), "hx_gemm_i8 i32") &&
            rc_ok(hx_gemm_i8(&ma, &mb, HX_LAYOUT_NK, &msa, &msb, &m16, HX_F16, s), "hx_gemm_i8 f16") &&
            hip_ok(hipStreamSynchronize(s), "sync");
  if (ok) {
    std::vector<int32_t> want(M * N);
    hxo_gemm_i8_i32(a.data(), K, bt.data(), K, 1, want.data(), N, M, N, K);
    std::vector<uint16_t> want16(M * N);
    hxo_dequant_i32_f16(want.data(), N, sa.data(), sb.data(), want16.data(), N, M, N);
    const auto got = d32.get();
    const auto got16 = d16.get();
    if (std::memcmp(got.data(), want.data(), got.size() * 4) != 0) {
      std::printf("FAIL gemm_i8: int32 result differs from the oracle\n");
      ok = false;
    }
    if (std::memcmp(got16.data(), want16.data(), got16.size() * 2) != 0) {
      std::printf("FAIL gemm_i8: fp16 dequant differs from the oracle bit for bit\n");
      ok = false;
    }
  }
  report(ok, "gemm_i8_i32_and_dequant_bitexact_512x384x640");
}

// C4-shaped row ops (fewer rows): softmax and RMSNorm on fp16 N(0, 2).
static void case_rows(hipStream_t s) {
  const int64_t R = 64, C = 4096;
  auto x = f16_vec(R * C, [] { return normal(2.f); });
  auto gamma = f16_vec(C, [] { return 1.f + normal(0.1f); });
  DevBuf<uint16_t> dx(x), dg(gamma), dy(R * C), dz(R * C);
  hx_memref2d mx = to_hx(desc2(dx.p, R, C, C)), my = to_hx(desc2(dy.p, R, C, C)),
              mz = to_hx(desc2(dz.p, R, C, C));
  hx_memref1d mg = to_hx(desc1(dg.p, C));
  bool ok = rc_ok(hx_softmax(&mx, &my, HX_F16, s), "hx_softmax") &&
            rc_ok(hx_rmsnorm(&mx, &mg, 1e-6f, &mz, HX_F16, s), "hx_rmsnorm") &&
            hip_ok(hipStreamSynchronize(s), "sync");
  if (ok) {
    std::vector<uint16_t> ws(R * C), wr(R * C);
    hxo_softmax(x.data(), ws.data(), HX_F16, R, C, C, C);
    hxo_rmsnorm(x.data(), gamma.data(), 1e-6f, wr.data(), HX_F16, R, C, C, C);
    ok = close(dy.get(), ws, 1e-2f, 1e-5f, "softmax") && close(dz.get(), wr, 1e-2f, 1e-2f, "rmsnorm");
  }
  report(ok, "softmax_rmsnorm_64x4096");
}

// A registered int8 weight ([K][N], f16 per-channel scales) through the
// decode GEMV (M = 4), the C3 contract, plus the content-hash dedupe.
static void case_resident_gemv(hipStream_t s) {
  const int64_t M = 4, N = 1376, K = 4096;
  std::vector<int8_t> w(K * N);
  for (auto& v : w) v = (int8_t)((int)(splitmix64() % 255) - 127);
  auto sc = f16_vec(N, [] { return uniform(0.001f, 0.02f); });
  auto x = f16_vec(M * K, [] { return normal(1.f); });
  DevBuf<int8_t> dw(w);
  DevBuf<uint16_t> dsc(sc), dx(x), dy(M * N);
  hx_memref2d mw = to_hx(desc2(dw.p, K, N, N)), mx = to_hx(desc2(dx.p, M, K, K)),
              my = to_hx(desc2(dy.p, M, N, N));
  hx_memref1d ms = to_hx(desc1(dsc.p, N));
  hx_weight_t h1 = nullptr, h2 = nullptr;
  bool ok = rc_ok(hx_weight_register(&mw, HX_I8, HX_LAYOUT_KN, &ms, HX_F16, s, &h1), "hx_weight_register") &&
            rc_ok(hx_weight_register(&mw, HX_I8, HX_LAYOUT_KN, &ms, HX_F16, s, &h2), "hx_weight_register again");
  if (ok && h1 != h2) {
    std::printf("FAIL resident: identical content registered twice gave two handles\n");
    ok = false;
  }
  int64_t k = 0, n = 0;
  int dt = 0, rc = 0;
  uint64_t hash = 0;
  ok = ok && rc_ok(hx_weight_info(h1, &k, &n, &dt, &hash, &rc), "hx_weight_info");
  if (ok && (k != K || n != N || dt != HX_I8 || rc != 2)) {
    std::printf("FAIL resident: info K=%lld N=%lld dtype=%d refcount=%d\n", (long long)k, (long long)n, dt, rc);
    ok = false;
  }
  ok = ok && rc_ok(hx_matmul_resident(&mx, HX_F16, h1, nullptr, 0, &my, HX_F16, s), "hx_matmul_resident") &&
       hip_ok(hipStreamSynchronize(s), "sync");
  if (ok) {
    std::vector<float> scf(N);
    for (int64_t j = 0; j < N; ++j) scf[j] = hxo_f16_to_f32(sc[j]);
    std::vector<uint16_t> want(M * N);
    hxo_matmul(x.data(), HX_F16, K, w.data(), HX_I8, N, 0, scf.data(), nullptr, 0, 0, want.data(), HX_F16, N, M,
               N, K);
    ok = close(dy.get(), want, 1e-2f, 1e-3f, "resident gemv");
  }
  if (h2) ok = rc_ok(hx_weight_release(h2), "hx_weight_release") && ok;
  if (h1) ok = rc_ok(hx_weight_release(h1), "hx_weight_release") && ok;
  if (ok && hx_weight_info(h1, &k, &n, &dt, &hash, &rc) != HX_ERR_HANDLE) {
    std::printf("FAIL resident: a released handle is still known\n");
    ok = false;
  }
  report(ok, "resident_w8a16_gemv_4x1376x4096");
}

// The native tuner from C++: tune the int8 family at one shape, pin the
// champion, check the pinned call is still exact, and round-trip the pins.
static void case_tune(hipStream_t s) {
  const int64_t M = 512, N = 512, K = 512;
  hx_tune_options opt;
  std::memset(&opt, 0, sizeof opt);
  opt.reps = 3;
  opt.budget_us = 5000.0;
  opt.min_iters = 5;
  opt.max_iters = 50;
  opt.pin = 1;
  opt.canary_reference_us = -1.0;  // this round sets the canary reference
  static hx_tune_report rep;
  bool ok = rc_ok(hx_tune(HX_OP_GEMM_I8, M, N, K, &opt, &rep, s), "hx_tune");
  int idx = -1;
  ok = ok && rc_ok(hx_config_lookup(HX_OP_GEMM_I8, M, N, K, &idx), "hx_config_lookup");
  if (ok && (rep.champion_index < 0 || !rep.round_valid || idx != rep.champion_index)) {
    std::printf("FAIL tune: champion %d valid %d pinned lookup %d\n", rep.champion_index, rep.round_valid, idx);
    ok = false;
  }
  hx_kernel_config cfg;
  ok = ok && rc_ok(hx_config_get(HX_OP_GEMM_I8, idx, &cfg), "hx_config_get");
  if (ok) {
    std::vector<int8_t> a(M * K), bt(N * K);
    for (auto& v : a) v = (int8_t)((int)(splitmix64() % 255) - 127);
    for (auto& v : bt) v = (int8_t)((int)(splitmix64() % 255) - 127);
    DevBuf<int8_t> da(a), db(bt);
    DevBuf<int32_t> dc(M * N);
    hx_memref2d ma = to_hx(desc2(da.p, M, K, K)), mb = to_hx(desc2(db.p, N, K, K)),
                mc = to_hx(desc2(dc.p, M, N, N));
    ok = rc_ok(hx_gemm_i8(&ma, &mb, HX_LAYOUT_NK, nullptr, nullptr, &mc, HX_I32, s), "hx_gemm_i8 pinned") &&
         hip_ok(hipStreamSynchronize(s), "sync");
    if (ok) {
      std::vector<int32_t> want(M * N);
      hxo_gemm_i8_i32(a.data(), K, bt.data(), K, 1, want.data(), N, M, N, K);
      const auto got = dc.get();
      if (std::memcmp(got.data(), want.data(), got.size() * 4) != 0) {
        std::printf("FAIL tune: the pinned champion %s is not exact\n", cfg.name);
        ok = false;
      }
    }
  }
  size_t need = 0;
  (void)hx_config_pins_save(nullptr, 0, &need);  // HX_ERR_ARG, with the size needed
  std::string text(need, '\0');
  ok = ok && rc_ok(hx_config_pins_save(&text[0], text.size(), &need), "hx_config_pins_save");
  ok = ok && rc_ok(hx_config_select(HX_OP_GEMM_I8, M, N, K, -1), "hx_config_select -1") &&
       rc_ok(hx_config_pins_load(text.c_str()), "hx_config_pins_load");
  int idx2 = -2;
  ok = ok && rc_ok(hx_config_lookup(HX_OP_GEMM_I8, M, N, K, &idx2), "hx_config_lookup after load");
  if (ok && idx2 != idx) {
    std::printf("FAIL tune: pins text did not restore the champion (%d against %d)\n", idx2, idx);
    ok = false;
  }
  (void)hx_config_select(HX_OP_GEMM_I8, M, N, K, -1);
  if (ok) std::printf("tune: champion %s, control q50 %.2f us, best q50 %.2f us\n", cfg.name, rep.control_q50_us,
                      rep.best_q50_us);
  report(ok, "hx_tune_gemm_i8_512_pin_and_pins_roundtrip");
}

// Errors come back as codes with a reason; nothing is enqueued.
static void case_errors(hipStream_t s) {
  const int64_t M = 64, N = 64, K = 128;
  DevBuf<int8_t> da(M * K), db(N * (K + 16));
  DevBuf<int32_t> dc(M * N);
  hx_memref2d ma = to_hx(desc2(da.p, M, K, K)), mb = to_hx(desc2(db.p, N, K + 16, K + 16)),
              mc = to_hx(desc2(dc.p, M, N, N));
  const int rc = hx_gemm_i8(&ma, &mb, HX_LAYOUT_NK, nullptr, nullptr, &mc, HX_I32, s);
  bool ok = rc == HX_ERR_SHAPE && std::strlen(hx_last_error()) > 0;
  if (!ok) std::printf("FAIL errors: K mismatch returned %d (%s)\n", rc, hx_last_error());
  const int rc2 = hx_softmax(&mc, &mc, HX_I32, s);
  if (rc2 != HX_ERR_DTYPE) {
    std::printf("FAIL errors: int32 softmax returned %d\n", rc2);
    ok = false;
  }
  report(ok, "error_codes");
}

int main() {
  if (hx_init() != HX_OK) {
    std::printf("FAIL hx_init: %s\n", hx_last_error());
    return 1;
  }
  std::printf("build %s\n", hx_build_id());
  hipStream_t s;
  if (!hip_ok(hipStreamCreate(&s), "hipStreamCreate")) return 1;
  case_matmul_residual(s);
  case_gemm_i8(s);
  case_rows(s);
  case_resident_gemv(s);
  case_tune(s);
  case_errors(s);
  (void)hipStreamDestroy(s);
  if (g_failed == 0) std::printf("ALL PASS\n");
  return g_failed == 0 ? 0 : 1;
}
