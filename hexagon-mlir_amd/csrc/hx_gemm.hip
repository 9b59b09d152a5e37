// hx_gemm.hip -- dispatch of the MFMA GEMM family (config tables, untuned
// default choice, fast-path preconditions) and the generic any-shape kernel.
// The tiled kernel template is in hx_gemm_kernel.hpp; its per-mode config
// tables are in hx_gemm_{i8,f16,bf16,w8}.hip.
#include "hx_gemm_kernel.hpp"

#include <algorithm>
#include <atomic>

namespace hx {

// ---------------------------------------------------------------------------
// Generic kernel: any shape, any alignment, same arithmetic contract (int32
// exact for GM_I8; binary32 accumulation otherwise).  One 256-thread block
// computes a 32x32 tile, each thread 4 outputs, K staged 32 at a time in LDS.
// ---------------------------------------------------------------------------
template <int MODE, int EPI>
__global__ void __launch_bounds__(256) gemm_generic_kernel(GemmArgs p) {
  typedef ModeTraits<MODE> T;
  constexpr int NB = (EPI == GE_SWIGLU) ? 2 : 1;
  __shared__ float sa[32][33];
  __shared__ float sb[NB][32][33];
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // ty 0..7
  const int64_t m0 = (int64_t)blockIdx.y * 32, n0 = (int64_t)blockIdx.x * 32;
  typedef typename std::conditional<MODE == GM_I8, int, float>::type AccT;
  AccT acc[NB][4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[nb][q] = 0;
  for (int64_t k0 = 0; k0 < p.K; k0 += 32) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r = ty + 8 * q;
      const int64_t gm = m0 + r, gk = k0 + tx;
      float av = 0.f;
      if (gm < p.M && gk < p.K) {
        if constexpr (MODE == GM_I8) av = (float)reinterpret_cast<const int8_t*>(p.a)[gm * p.lda + gk];
        else if constexpr (MODE == GM_BF16) av = bf16_to_f32(reinterpret_cast<const uint16_t*>(p.a)[gm * p.lda + gk]);
        else av = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p.a)[gm * p.lda + gk]);
      }
      sa[r][tx] = av;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const void* bp = nb == 0 ? p.b : p.b2;
        const int64_t gn = n0 + r;
        float bv = 0.f;
        if (gn < p.N && gk < p.K) {
          if constexpr (T::EB == 1) bv = (float)reinterpret_cast<const int8_t*>(bp)[gn * p.ldb + gk];
          else if constexpr (MODE == GM_BF16) bv = bf16_to_f32(reinterpret_cast<const uint16_t*>(bp)[gn * p.ldb + gk]);
          else bv = f16_bits_to_f32(reinterpret_cast<const uint16_t*>(bp)[gn * p.ldb + gk]);
        }
        sb[nb][r][tx] = bv;
      }
    }
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < 32; ++kk)
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          if constexpr (MODE == GM_I8)
            acc[nb][q] += (int)sa[ty + 8 * q][kk] * (int)sb[nb][tx][kk];
          else
            acc[nb][q] = acc[nb][q] + sa[ty + 8 * q][kk] * sb[nb][tx][kk];
        }
    __syncthreads();
  }
  const int64_t col = n0 + tx;
  if (col >= p.N) return;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int64_t row = m0 + ty + 8 * q;
    if (row >= p.M) continue;
    const int64_t idx = row * p.ldc + col;
    if constexpr (MODE == GM_I8) {
      if (p.out_dtype == DT_I32) {
        reinterpret_cast<int*>(p.c)[idx] = acc[0][q];
      } else {
        float t = (float)acc[0][q];
        if (p.row_scale) t = t * p.row_scale[row];
        if (p.col_scale) t = t * p.col_scale[col];
        store_out(p.c, p.out_dtype, idx, t);
      }
    } else if constexpr (EPI == GE_SWIGLU) {
      const float cs = p.col_scale ? p.col_scale[col] : 1.f;
      const float cs2 = p.col_scale2 ? p.col_scale2[col] : 1.f;
      const float g = f16_bits_to_f32(f32_to_f16_bits(acc[0][q] * cs));
      const float u = f16_bits_to_f32(f32_to_f16_bits(acc[NB - 1][q] * cs2));
      const float sg = g / (1.0f + fast_exp(-g));
      reinterpret_cast<uint16_t*>(p.c)[idx] = f32_to_f16_bits(sg * u);
    } else {
      float t = acc[0][q];
      if (p.col_scale) t = t * p.col_scale[col];
      if (p.res) t = t + load_any(p.res, p.res_dtype, row * p.ldr + col);
      store_out(p.c, p.out_dtype, idx, t);
    }
  }
}

static const GemmEntry* table(int mode, int& n) {
  switch (mode) {
    case GM_I8: return gemm_table_i8(n);
    case GM_F16: return gemm_table_f16(n);
    case GM_BF16: return gemm_table_bf16(n);
    case GM_W8: return gemm_table_w8(n);
    default: n = 0; return nullptr;
  }
}

int gemm_config_count(int mode) {
  int n;
  table(mode, n);
  return n;
}

const GemmConfig* gemm_config(int mode, int idx) {
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t || idx < 0 || idx >= n) return nullptr;
  return &t[idx].cfg;
}

int gemm_num_cus();
// CU count of the device (read once; every thread that races to read it
// stores the same value).
static std::atomic<int> g_num_cus{0};
static int num_cus() {
  int n = g_num_cus.load(std::memory_order_relaxed);
  if (n == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      n = v;
    else
      n = 256;
    g_num_cus.store(n, std::memory_order_relaxed);
  }
  return n;
}
int gemm_num_cus() { return num_cus(); }

// The clock hook's per-device counters (null: off).  Launching threads read
// them while the API thread sets them, hence atomics.
static std::atomic<unsigned long long*> g_clk[64];
static std::atomic<int> g_clk_on{0};
void gemm_clock_target(int dev, unsigned long long* clk) {
  if (dev < 0 || dev >= 64) return;
  g_clk[dev].store(clk, std::memory_order_release);
  int on = 0;
  for (int d = 0; d < 64; ++d) on |= g_clk[d].load(std::memory_order_relaxed) != nullptr;
  g_clk_on.store(on, std::memory_order_release);
}
static unsigned long long* clock_target() {
  if (!g_clk_on.load(std::memory_order_acquire)) return nullptr;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  return g_clk[dev].load(std::memory_order_acquire);
}

// Untuned choice: estimated time = rounds * occ * tile_area / rate, where a
// round is one workgroup in every resident slot (CUs x occ).  The autotuner
// replaces this guess per shape.
int gemm_default_config(int mode, int epi, int64_t M, int64_t N, int64_t K) {
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t) return -1;
  const int cus = num_cus();
  int best = -1;
  double best_cost = 0;
  // Cost: the tiles of the busiest CU times one tile's area over the
  // config's relative per-CU rate (tiles sharing a CU split its rate),
  // divided by an occupancy efficiency sqrt(resident / occ): a CU holding
  // fewer workgroups than it can is latency-bound (one 64x64 tile per CU ran
  // at half speed).  A K split runs ksplit workgroups per tile on 1/ksplit
  // of K each, plus a merge (x1.5, x1.05 from K = 8192 on, where the merge
  // is small against the product), and needs >= 512 k per part.  Counting
  // occupancy-limited rounds instead picked 64x64 at 2048^3, where 128x128
  // measured 1.2-1.4x faster (f16 and int8).
  const int64_t ea = mode == GM_I8 ? 1 : 2;
  // first pass: configs whose LDS ring K fills (at least as many K stages
  // per part, the last one partial, as the ring holds); when K is shorter
  // than every ring, a second pass takes any unsplit config
  for (int pass = 0; pass < 2 && best < 0; ++pass)
  for (int i = 0; i < n; ++i) {
    const GemmConfig& c = t[i].cfg;
    if (c.epi != epi) continue;
    const int ks = c.ksplit > 1 ? c.ksplit : 1;
    if (ks > 1 && (pass == 1 || K / ks < 512)) continue;
    if (pass == 0 && (K / ks * ea + c.sb - 1) / c.sb < c.stages) continue;
    const int64_t tiles = ((M + c.bm - 1) / c.bm) * ((N + c.bn - 1) / c.bn) * ks;
    const int64_t per_cu_i = (tiles + cus - 1) / cus;
    const double per_cu = (double)per_cu_i;
    const double resident = (double)(per_cu_i < c.occ ? per_cu_i : c.occ);
    const double eff = sqrt(resident / (double)c.occ);
    const double merge = ks > 1 ? (K >= 8192 ? 1.05 : 1.5) : 1.0;
    const double cost = per_cu * (double)c.bm * c.bn / c.rate / ks / eff * merge;
    if (best < 0 || cost < best_cost - 1e-9) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

const char* gemm_fast_refusal(int mode, const GemmArgs& a) {
  const int ea = (mode == GM_I8) ? 1 : 2;
  const int eb = (mode == GM_I8 || mode == GM_W8) ? 1 : 2;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return "empty";
  if (!al16(a.a) || !al16(a.b) || (a.b2 && !al16(a.b2))) return "unaligned-base";
  if ((a.lda * ea) % 16 != 0 || (a.ldb * eb) % 16 != 0) return "row-stride";
  if ((a.K * ea) % 16 != 0 || (a.K * eb) % 16 != 0) return "k-granularity";
  // 32-bit buffer offsets inside one tile's row range (operands and output)
  if ((int64_t)256 * a.lda * ea >= ((int64_t)1 << 31)) return "offset-range";
  if ((int64_t)256 * a.ldc * 4 >= ((int64_t)1 << 31)) return "offset-range";
  if (a.b_kn) {
    // [K][N] B (int8, f16, bf16): whole 16-byte chunks of a row, every row
    // of k addressed with 32-bit offsets
    if (mode != GM_F16 && mode != GM_BF16 && mode != GM_I8) return "b-layout";
    if ((a.N * eb) % 16 != 0) return "n-granularity";
    if (a.K * a.ldb * eb >= ((int64_t)1 << 31)) return "offset-range";
  } else if ((int64_t)256 * a.ldb * eb >= ((int64_t)1 << 31)) {
    return "offset-range";
  }
  // at least one 32-byte MFMA k-step of A per row.  K shorter than a
  // config's stage ring is fine: the ring's extra stages load zeros through
  // the buffer range (every config is tested exact at K below its ring),
  // which for small K still beats the generic kernel by 3x.
  if (a.K * ea < 32) return "shallow-k";
  // the epilogue stores (and reads the residual as) four consecutive outputs
  if (a.N % 4 != 0) return "n-granularity";
  if (a.ldc % 4 != 0 || !al16(a.c)) return "output-layout";
  if (a.res && (a.ldr % 4 != 0 || !al16(a.res))) return "residual-layout";
  return nullptr;
}

bool gemm_fast_ok(int mode, const GemmArgs& a) { return gemm_fast_refusal(mode, a) == nullptr; }

// Merge of a K split: y[m][n] = RNE((sum_s part[s][m][n]) * col_scale[n]
// (+ residual[m][n])), parts summed in order; four columns per thread
// (N % 4 == 0 on the tiled path).
// Eight columns per thread with 16-byte loads and stores (N, ldc and ldr
// multiples of 8, 16-byte aligned column scales): OUT is the output type,
// the residual's type is a uniform branch.
template <int OUT>
__global__ void __launch_bounds__(256) splitk_merge8_kernel(GemmArgs a, const float* part, int parts) {
  const uint32_t q = blockIdx.x * 256u + threadIdx.x;
  const uint32_t n8 = (uint32_t)(a.N >> 3);
  if (q >= (uint32_t)a.M * n8) return;
  const uint32_t m = q / n8;
  const int64_t n = 8 * (int64_t)(q - m * n8);
  const int64_t mn = a.M * a.N;
  const float* p = part + (int64_t)m * a.N + n;
  v4f lo = v4f{0.f, 0.f, 0.f, 0.f}, hi = lo;
  for (int s = 0; s < parts; ++s) {
    lo += *reinterpret_cast<const v4f*>(p + s * mn);
    hi += *reinterpret_cast<const v4f*>(p + s * mn + 4);
  }
  float v[8] = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  if (a.col_scale) {
    const v4f s0 = *reinterpret_cast<const v4f*>(a.col_scale + n);
    const v4f s1 = *reinterpret_cast<const v4f*>(a.col_scale + n + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) { v[i] = v[i] * s0[i]; v[i + 4] = v[i + 4] * s1[i]; }
  }
  if (a.res) {
    const int64_t r = (int64_t)m * a.ldr + n;
    if (a.res_dtype == DT_F32) {
      const v4f r0 = *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(a.res) + r);
      const v4f r1 = *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(a.res) + r + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { v[i] = v[i] + r0[i]; v[i + 4] = v[i + 4] + r1[i]; }
    } else {
      const v4i rr = *reinterpret_cast<const v4i*>(reinterpret_cast<const uint16_t*>(a.res) + r);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint16_t h = (uint16_t)((uint32_t)rr[i >> 1] >> (16 * (i & 1)));
        v[i] = v[i] + (a.res_dtype == DT_F16 ? f16_bits_to_f32(h) : bf16_to_f32(h));
      }
    }
  }
  const int64_t o = (int64_t)m * a.ldc + n;
  if constexpr (OUT == DT_F32) {
    *reinterpret_cast<v4f*>(reinterpret_cast<float*>(a.c) + o) = v4f{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<v4f*>(reinterpret_cast<float*>(a.c) + o + 4) = v4f{v[4], v[5], v[6], v[7]};
  } else {
    v4i w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t l = OUT == DT_F16 ? f32_to_f16_bits(v[2 * i]) : f32_to_bf16(v[2 * i]);
      const uint32_t h = OUT == DT_F16 ? f32_to_f16_bits(v[2 * i + 1]) : f32_to_bf16(v[2 * i + 1]);
      w[i] = (int)(l | (h << 16));
    }
    *reinterpret_cast<v4i*>(reinterpret_cast<uint16_t*>(a.c) + o) = w;
  }
}

__global__ void __launch_bounds__(256) splitk_merge_kernel(GemmArgs a, const float* part, int parts) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n4 = a.N / 4;
  if (q >= a.M * n4) return;
  const int64_t m = q / n4, n = 4 * (q - m * n4);
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < parts; ++s)
    acc += *reinterpret_cast<const v4f*>(part + ((int64_t)s * a.M + m) * a.N + n);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v = acc[i];
    if (a.col_scale) v = v * a.col_scale[n + i];
    if (a.res) v = v + load_any(a.res, a.res_dtype, m * a.ldr + n + i);
    store_out(a.c, a.out_dtype, m * a.ldc + n + i, v);
  }
}

// Merge of an int8 K split: the int32 partials summed in order with
// two's-complement wrap-around (integer addition is associative, so the sum
// equals the unsplit accumulator bit for bit), then the fused epilogue's
// dequant ((float)acc * row_scale) * col_scale, an absent scale reading as
// 1.0, rounded to the output type; DT_I32 stores the sum.  Four columns per
// thread with 16-byte partial loads (N % 4 == 0 on the tiled path).
template <int OUT>
__global__ void __launch_bounds__(256) splitk_merge_i8_kernel(GemmArgs a, const int* part, int parts) {
  const uint32_t q = blockIdx.x * 256u + threadIdx.x;
  const uint32_t n4 = (uint32_t)(a.N >> 2);
  if (q >= (uint32_t)a.M * n4) return;
  const uint32_t m = q / n4;
  const int64_t n = 4 * (int64_t)(q - m * n4);
  const int64_t mn = a.M * a.N;
  const int* p = part + (int64_t)m * a.N + n;
  uint32_t acc[4] = {0u, 0u, 0u, 0u};
  for (int s = 0; s < parts; ++s) {
    const v4i v = *reinterpret_cast<const v4i*>(p + s * mn);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += (uint32_t)v[i];
  }
  const int64_t o = (int64_t)m * a.ldc + n;
  if constexpr (OUT == DT_I32) {
    *reinterpret_cast<v4i*>(reinterpret_cast<int*>(a.c) + o) =
        v4i{(int)acc[0], (int)acc[1], (int)acc[2], (int)acc[3]};
  } else {
    const float rs = a.row_scale ? a.row_scale[m] : 1.f;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float cs = a.col_scale ? a.col_scale[n + i] : 1.f;
      v[i] = ((float)(int)acc[i] * rs) * cs;
    }
    if constexpr (OUT == DT_F32) {
      *reinterpret_cast<v4f*>(reinterpret_cast<float*>(a.c) + o) = v4f{v[0], v[1], v[2], v[3]};
    } else if constexpr (OUT == DT_BF16) {
      const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
      *reinterpret_cast<v2i*>(reinterpret_cast<uint16_t*>(a.c) + o) = v2i{(int)lo, (int)hi};
    } else {
      *reinterpret_cast<v2i*>(reinterpret_cast<uint16_t*>(a.c) + o) =
          v2i{(int)f32x2_to_f16x2(v[0], v[1]), (int)f32x2_to_f16x2(v[2], v[3])};
    }
  }
}

// K elements of one part of a split: whole K stages of the config's width
// per part (an int8 stage is sb elements, a 16-bit one sb / 2).
static int64_t split_k_elems(int mode, const GemmConfig& c, const GemmArgs& a) {
  const int64_t bke = mode == GM_I8 ? c.sb : c.sb / 2;
  const int64_t per = (a.K + c.ksplit - 1) / c.ksplit;
  return (per + bke - 1) / bke * bke;
}

// Partials of a split launch: [parts][M][N] for the merge kernel, or
// [parts][tiles][BM*BN] for the merge inside the kernel; the larger of the
// two (they differ on edge tiles), binary32 or int32.
size_t gemm_part_bytes(int mode, int cfg_idx, const GemmArgs& a) {
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t || cfg_idx < 0 || cfg_idx >= n || t[cfg_idx].cfg.ksplit <= 1) return 0;
  const GemmConfig& c = t[cfg_idx].cfg;
  const int64_t ks = split_k_elems(mode, c, a);
  const int64_t parts = (a.K + ks - 1) / ks;
  const int64_t tiles = ((a.M + c.bm - 1) / c.bm) * ((a.N + c.bn - 1) / c.bn);
  const int64_t per = std::max<int64_t>(a.M * a.N, tiles * c.bm * c.bn);
  return (size_t)parts * (size_t)per * sizeof(float);
}

int64_t gemm_tiles(int mode, int cfg_idx, const GemmArgs& a) {
  const GemmConfig* c = gemm_config(mode, cfg_idx);
  return c ? ((a.M + c->bm - 1) / c->bm) * ((a.N + c->bn - 1) / c->bn) : 0;
}

int launch_gemm(int mode, int cfg_idx, const GemmArgs& a, hipStream_t s) {
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t || cfg_idx < 0 || cfg_idx >= n) return HXI_ERR_ARG;
  const GemmConfig& c = t[cfg_idx].cfg;
  const int64_t tiles = ((a.M + c.bm - 1) / c.bm) * ((a.N + c.bn - 1) / c.bn);
  if (tiles <= 0 || tiles > 0x7fffffff) return HXI_ERR_SHAPE;
  if (c.ksplit <= 1) {
    GemmArgs q = a;
    q.k_split = 0;
    q.cnt = nullptr;
    q.clk = clock_target();
    t[cfg_idx].fn(q, s);
    return HXI_OK;
  }
  if (a.b2 || !a.part || (mode != GM_I8 && a.row_scale)) return HXI_ERR_ARG;
  // K split with counters: the parts of each tile hand their partials to
  // the last of them, which applies the epilogue -- one launch (B as
  // [N][K], or [K][N] read in place)
  if (a.cnt && tiles <= kGemvSplitCounters) {
    GemmArgs q = a;
    q.k_split = split_k_elems(mode, c, a);
    q.clk = clock_target();
    t[cfg_idx].fn(q, s);
    return HXI_OK;
  }
  // K split without counters: binary32 (int8: int32) partials into a.part,
  // then a merge kernel applies the epilogue (scales, residual, rounding)
  GemmArgs q = a;
  q.cnt = nullptr;
  q.clk = clock_target();
  q.k_split = split_k_elems(mode, c, a);
  q.c = a.part;
  q.ldc = a.N;
  q.out_dtype = mode == GM_I8 ? DT_I32 : DT_F32;
  q.row_scale = nullptr;
  q.col_scale = nullptr;
  q.res = nullptr;
  const int parts = (int)((a.K + q.k_split - 1) / q.k_split);
  t[cfg_idx].fn(q, s);
  if (mode == GM_I8) {
    if ((uint64_t)a.M * (uint64_t)(a.N / 4) >= ((uint64_t)1 << 32)) return HXI_ERR_SHAPE;
    const dim3 grid((unsigned)((a.M * (a.N / 4) + 255) / 256));
    const int* ip = reinterpret_cast<const int*>(a.part);
    switch (a.out_dtype) {
      case DT_I32: splitk_merge_i8_kernel<DT_I32><<<grid, dim3(256), 0, s>>>(a, ip, parts); break;
      case DT_F32: splitk_merge_i8_kernel<DT_F32><<<grid, dim3(256), 0, s>>>(a, ip, parts); break;
      case DT_BF16: splitk_merge_i8_kernel<DT_BF16><<<grid, dim3(256), 0, s>>>(a, ip, parts); break;
      default: splitk_merge_i8_kernel<DT_F16><<<grid, dim3(256), 0, s>>>(a, ip, parts); break;
    }
    return HXI_OK;
  }
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool v8 = a.N % 8 == 0 && a.ldc % 8 == 0 && (!a.res || a.ldr % 8 == 0) &&
                  (!a.col_scale || al16(a.col_scale)) && a.M * (a.N / 8) < ((int64_t)1 << 31) &&
                  (a.out_dtype == DT_F16 || a.out_dtype == DT_BF16 || a.out_dtype == DT_F32);
  if (v8) {
    const dim3 grid((unsigned)((a.M * (a.N / 8) + 255) / 256));
    if (a.out_dtype == DT_F16) splitk_merge8_kernel<DT_F16><<<grid, dim3(256), 0, s>>>(a, a.part, parts);
    else if (a.out_dtype == DT_BF16) splitk_merge8_kernel<DT_BF16><<<grid, dim3(256), 0, s>>>(a, a.part, parts);
    else splitk_merge8_kernel<DT_F32><<<grid, dim3(256), 0, s>>>(a, a.part, parts);
    return HXI_OK;
  }
  const int64_t threads = a.M * (a.N / 4);
  splitk_merge_kernel<<<dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s>>>(a, a.part, parts);
  return HXI_OK;
}

int launch_gemm_generic(int mode, const GemmArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.N + 31) / 32), (unsigned)((a.M + 31) / 32));
  const bool sw = a.b2 != nullptr;
  switch (mode) {
    case GM_I8: gemm_generic_kernel<GM_I8, GE_STORE><<<grid, dim3(256), 0, s>>>(a); break;
    case GM_F16: gemm_generic_kernel<GM_F16, GE_STORE><<<grid, dim3(256), 0, s>>>(a); break;
    case GM_BF16: gemm_generic_kernel<GM_BF16, GE_STORE><<<grid, dim3(256), 0, s>>>(a); break;
    case GM_W8:
      if (sw) gemm_generic_kernel<GM_W8, GE_SWIGLU><<<grid, dim3(256), 0, s>>>(a);
      else gemm_generic_kernel<GM_W8, GE_STORE><<<grid, dim3(256), 0, s>>>(a);
      break;
    default: return HXI_ERR_ARG;
  }
  return HXI_OK;
}

}  // namespace hx
