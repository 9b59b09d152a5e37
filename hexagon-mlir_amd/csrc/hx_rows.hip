// hx_rows.hip -- single-pass row reductions over the last dimension:
// softmax, RMSNorm and LayerNorm, plus the elementwise SiLU*mul of the FFN.
//
// Reference semantics (hexagon-mlir paths, QHB = qcom_hexagon_backend):
//   softmax   docs/tutorials/torch-mlir/softmax.md:178-226,
//             test/python/triton/test_softmax.py:41-69, DivToMul
//             (QHB/lib/Transforms/DivToMulOptimizationPass.cpp:9-18)
//   RMSNorm   test/python/triton/test_rms_norm.py:34-59, FastInverse
//             (QHB/lib/Transforms/FastInversePass.cpp:97-140)
//   LayerNorm test/python/triton/test_layer_norm.py:39-79
// The reference folds each row 128 bytes at a time on HVX and finishes with a
// log2(lanes) rotate-and-fold (QHB/lib/Conversion/LinalgToLLVM/
// VectorRowReducePass.cpp:17-28).  Here a row is held in VGPRs by one wave
// (rows up to 4 KiB) or by the four waves of a workgroup (longer rows):
// every element is read from HBM once with 16-byte loads and written once,
// and the reductions are 64-lane butterflies (plus one LDS exchange when
// four waves share a row).
// All arithmetic is binary32 with one rounding to the storage type.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

enum RowOp : int { ROW_SOFTMAX = 0, ROW_RMSNORM = 1, ROW_LAYERNORM = 2 };

struct RowArgs {
  const void* x; int64_t ldx;
  void* y; int64_t ldy;
  const void* w;   // gamma (RMSNorm) / weight (LayerNorm), may be null
  const void* b;   // LayerNorm bias, may be null
  float* mean;     // LayerNorm per-row outputs, may be null
  float* rstd;
  float eps;
  int64_t rows, cols;
};

// Sum / max across the WPR waves of a workgroup that share one row.
template <int WPR>
__device__ __forceinline__ float group_sum(float v, float* red) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();  // the previous use of `red` is finished everywhere
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) s += red[i];
    return s;
  }
}
// group_sum for a buffer this workgroup has not used before: no barrier
// guards a previous use, so one barrier (the publish) remains.
template <int WPR>
__device__ __forceinline__ float group_sum_once(float v, float* red) {
  v = wave_sum(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) s += red[i];
    return s;
  }
}
template <int WPR>
__device__ __forceinline__ float group_max(float v, float* red) {
  v = wave_max(v);
  if constexpr (WPR == 1) {
    return v;
  } else {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) m = fmaxf(m, red[i]);
    return m;
  }
}

// One kernel template for the three ops.
//   DT   storage dtype (f16 / bf16 / f32)
//   WPR  waves per row (1: a 256-thread block handles 4 rows; 4: one row)
//   VPL  16-byte vectors per lane
//   VEC  true when rows are 16-byte aligned and cols is a multiple of the
//        vector width, so whole vectors are loaded; false loads element by
//        element with a mask.
// Column of element e of vector v in lane l of wave w (of the row's group):
//   ((v * WPR + w) * 64 + l) * EV + e
// so every load instruction of a wave covers 1 KiB of contiguous row.
template <int OP, int DT, int WPR, int VPL, bool VEC>
__global__ void __launch_bounds__(256) row_kernel(RowArgs a) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  constexpr int N = VPL * EV;
  __shared__ float red[4];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rows_per_block = 4 / WPR;
  const int wave_in_row = (WPR == 1) ? 0 : wave;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + (WPR == 1 ? wave : 0);
  if (row >= a.rows) return;  // uniform per wave; WPR==4 blocks have row < rows
  const int64_t cols = a.cols;
  const S* xr = reinterpret_cast<const S*>(a.x) + row * a.ldx;
  S* yr = reinterpret_cast<S*>(a.y) + row * a.ldy;

  float v[N];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c0 = ((int64_t)(i * WPR + wave_in_row) * 64 + lane) * EV;
    if constexpr (VEC) {
      if (c0 < cols) {
        const v4u raw = *reinterpret_cast<const v4u*>(xr + c0);
        const S* e = reinterpret_cast<const S*>(&raw);
#pragma unroll
        for (int j = 0; j < EV; ++j) v[i * EV + j] = Elem<DT>::load(e[j]);
      } else {
#pragma unroll
        for (int j = 0; j < EV; ++j) v[i * EV + j] = 0.f;
      }
    } else {
#pragma unroll
      for (int j = 0; j < EV; ++j)
        v[i * EV + j] = (c0 + j < cols) ? Elem<DT>::load(xr[c0 + j]) : 0.f;
    }
  }
  auto valid = [&](int i, int j) -> bool {
    return ((int64_t)(i * WPR + wave_in_row) * 64 + lane) * EV + j < cols;
  };

  float scale = 1.f, shift = 0.f;
  if constexpr (OP == ROW_SOFTMAX) {
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < EV; ++j)
        if (valid(i, j)) m = fmaxf(m, v[i * EV + j]);
    m = group_max<WPR>(m, red);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < EV; ++j) {
        const float e = valid(i, j) ? fast_exp(v[i * EV + j] - m) : 0.f;
        v[i * EV + j] = e;
        s += e;
      }
    s = group_sum<WPR>(s, red);
    scale = 1.0f / s;  // DivToMul: one reciprocal, then multiplies
  } else if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) ss += v[k] * v[k];  // masked lanes hold 0
    ss = group_sum<WPR>(ss, red);
    scale = 1.0f / sqrtf(ss / (float)cols + a.eps);
  } else {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < N; ++k) s += v[k];
    s = group_sum<WPR>(s, red);
    const float mean = s / (float)cols;
    float vs = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < EV; ++j) {
        const float d = valid(i, j) ? v[i * EV + j] - mean : 0.f;
        vs += d * d;
      }
    vs = group_sum<WPR>(vs, red);
    scale = 1.0f / sqrtf(vs / (float)cols + a.eps);
    shift = mean;
    if ((int)threadIdx.x == (WPR == 1 ? wave * 64 : 0)) {
      if (a.mean) a.mean[row] = mean;
      if (a.rstd) a.rstd[row] = scale;
    }
  }

  const S* wp = reinterpret_cast<const S*>(a.w);
  const S* bp = reinterpret_cast<const S*>(a.b);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int64_t c0 = ((int64_t)(i * WPR + wave_in_row) * 64 + lane) * EV;
    S out[EV];
    S wv[EV], bv[EV];
    if constexpr (OP != ROW_SOFTMAX) {
      if (VEC && c0 < cols) {
        if (wp) *reinterpret_cast<v4u*>(wv) = *reinterpret_cast<const v4u*>(wp + c0);
        if (bp) *reinterpret_cast<v4u*>(bv) = *reinterpret_cast<const v4u*>(bp + c0);
      } else if (!VEC) {
#pragma unroll
        for (int j = 0; j < EV; ++j) {
          if (wp && c0 + j < cols) wv[j] = wp[c0 + j];
          if (bp && c0 + j < cols) bv[j] = bp[c0 + j];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < EV; ++j) {
      float r;
      if constexpr (OP == ROW_SOFTMAX) {
        r = v[i * EV + j] * scale;
      } else if constexpr (OP == ROW_RMSNORM) {
        r = v[i * EV + j] * scale;
        if (wp) r = r * Elem<DT>::load(wv[j]);
      } else {
        r = (v[i * EV + j] - shift) * scale;
        if (wp) r = r * Elem<DT>::load(wv[j]);
        if (bp) r = r + Elem<DT>::load(bv[j]);
      }
      out[j] = Elem<DT>::store(r);
    }
    if constexpr (VEC) {
      if (c0 < cols) *reinterpret_cast<v4u*>(yr + c0) = *reinterpret_cast<const v4u*>(out);
    } else {
#pragma unroll
      for (int j = 0; j < EV; ++j)
        if (c0 + j < cols) yr[c0 + j] = out[j];
    }
  }
}

// Vector path: rows are 16-byte aligned and cols is a multiple of the vector
// width.  The row stays in registers as raw 16-byte vectors (4 VGPRs per
// vector, independent of the element type) and is widened to binary32 on the
// fly in each pass, so a wave holding a 4096-wide fp16 row needs ~32 VGPRs
// for it and eight waves fit per SIMD: every row of an 8192-row problem is
// in flight at once.  Loads and stores are non-temporal (streamed once).
template <int DT>
__device__ __forceinline__ float vec_elem(const v4u& v, int j) {
  if constexpr (DT == DT_F32) {
    return __uint_as_float(v[j]);
  } else {
    const uint32_t w = v[j >> 1];
    const uint16_t h = (j & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
    return Elem<DT>::load(h);
  }
}

// 8-wave rows: each pass converts the raw vectors again.  Left to itself the
// compiler keeps the 256 converted binary32 elements per lane live across the
// reductions (for f16, spilling); an empty asm that may change the raw
// vectors makes every pass start from the 128 raw VGPRs (same values).
template <int VPL>
__device__ __forceinline__ void opaque_vecs(v4u (&raw)[VPL]) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) asm volatile("" : "+v"(raw[i]));
}

// The reduction and write-back of one row held in registers: raw holds the
// row's vectors, wv / bv gamma / beta at the same columns (zero where absent),
// red 2 * NRED floats that no other row in flight in this workgroup uses.
template <int OP, int DT, int WPR, int VPL, int NRED>
__device__ __forceinline__ void row_vec_finish(const RowArgs& a, int64_t row, int wave, int lane,
                                               v4u (&raw)[VPL], const v4u (&wv)[VPL],
                                               const v4u (&bv)[VPL], float* red) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  const int wave_in_row = (WPR == 1) ? 0 : wave;
  const int64_t cols = a.cols;
  S* yr = reinterpret_cast<S*>(a.y) + row * a.ldy;
  bool ok[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) ok[i] = ((int64_t)(i * WPR + wave_in_row) * 64 + lane) * EV < cols;

  // Softmax rows of at most 4 vectors per lane keep the exponentials of the
  // sum pass (binary32, 4 VGPRs per vector) and scale them in the output
  // pass instead of taking every exponential twice.
  constexpr bool KEEP_EXP = OP == ROW_SOFTMAX && VPL <= 4;
  float ex[KEEP_EXP ? VPL : 1][KEEP_EXP ? EV : 1];
  float scale = 1.f, shift = 0.f;
  if constexpr (OP == ROW_SOFTMAX) {
    // One exchange across the row's waves: each wave reduces its own max m_w
    // and sum s_w = sum exp(x - m_w), and the pairs combine as
    // m = max m_w, s = sum s_w exp(m_w - m) (the online-softmax merge,
    // test_online_softmax.py:28-78) -- one barrier per row instead of a max
    // exchange and a sum exchange (four barriers).
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (ok[i]) {
#pragma unroll
        for (int j = 0; j < EV; ++j) m = fmaxf(m, vec_elem<DT>(raw[i], j));
      }
    m = wave_max(m);
    if constexpr (WPR > 4) opaque_vecs<VPL>(raw);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (ok[i]) {
#pragma unroll
        for (int j = 0; j < EV; ++j) {
          const float e = fast_exp(vec_elem<DT>(raw[i], j) - m);
          if constexpr (KEEP_EXP) ex[i][j] = e;
          s += e;
        }
      }
    s = wave_sum(s);
    const float m_w = m;
    if constexpr (WPR > 1) {
      if (lane == 0) {
        red[wave] = m;
        red[NRED + wave] = s;
      }
      __syncthreads();
      float mg = red[0];
#pragma unroll
      for (int i = 1; i < WPR; ++i) mg = fmaxf(mg, red[i]);
      float sg = 0.f;
#pragma unroll
      for (int i = 0; i < WPR; ++i) sg += red[NRED + i] * fast_exp(red[i] - mg);
      m = mg;
      s = sg;
    }
    scale = 1.0f / s;  // DivToMul: one reciprocal, then multiplies
    shift = m;
    // kept exponentials are relative to this wave's own maximum:
    // exp(x - m) = exp(x - m_w) exp(m_w - m)
    if constexpr (KEEP_EXP && WPR > 1) scale = fast_exp(m_w - m) * scale;
  } else if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < EV; ++j) {
        const float v = vec_elem<DT>(raw[i], j);  // zero where not loaded
        ss += v * v;
      }
    ss = group_sum_once<WPR>(ss, red);
    scale = 1.0f / sqrtf(ss / (float)cols + a.eps);
  } else {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < EV; ++j) s += vec_elem<DT>(raw[i], j);
    s = group_sum_once<WPR>(s, red);
    const float mean = s / (float)cols;
    float vs = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (ok[i]) {
#pragma unroll
        for (int j = 0; j < EV; ++j) {
          const float d = vec_elem<DT>(raw[i], j) - mean;
          vs += d * d;
        }
      }
    vs = group_sum_once<WPR>(vs, red + NRED);
    scale = 1.0f / sqrtf(vs / (float)cols + a.eps);
    shift = mean;
    if ((int)threadIdx.x == (WPR == 1 ? wave * 64 : 0)) {
      if (a.mean) a.mean[row] = mean;
      if (a.rstd) a.rstd[row] = scale;
    }
  }

  if constexpr (WPR > 4) opaque_vecs<VPL>(raw);
  const bool has_w = a.w != nullptr, has_b = a.b != nullptr;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (!ok[i]) continue;
    const int64_t c0 = ((int64_t)(i * WPR + wave_in_row) * 64 + lane) * EV;
    S out[EV];
#pragma unroll
    for (int j = 0; j < EV; ++j) {
      const float x = vec_elem<DT>(raw[i], j);
      float r;
      if constexpr (KEEP_EXP) {
        r = ex[i][j] * scale;
      } else if constexpr (OP == ROW_SOFTMAX) {
        r = fast_exp(x - shift) * scale;
      } else if constexpr (OP == ROW_RMSNORM) {
        r = x * scale;
        if (has_w) r = r * vec_elem<DT>(wv[i], j);
      } else {
        r = (x - shift) * scale;
        if (has_w) r = r * vec_elem<DT>(wv[i], j);
        if (has_b) r = r + vec_elem<DT>(bv[i], j);
      }
      out[j] = Elem<DT>::store(r);
    }
    __builtin_nontemporal_store(*reinterpret_cast<const v4u*>(out), reinterpret_cast<v4u*>(yr + c0));
  }
}

// Loads of one row's vectors (and of gamma / beta at the same columns).
// Every load is a branch-free buffer load: chunks past the row end read zero
// from the descriptor's range, and a descriptor of zero bytes (a row past the
// end, or no gamma) reads zero without touching memory.  A load behind a
// per-lane test would make the compiler wait for it at the join.
template <int DT, int WPR, int VPL, int POLICY>
__device__ __forceinline__ void row_vec_load(const void* base, int64_t ld, int64_t row, int bytes,
                                             int wave_in_row, int lane, v4u (&dst)[VPL]) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  const S* p = reinterpret_cast<const S*>(base) + row * ld;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, bytes, 0x00020000);
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int off = ((i * WPR + wave_in_row) * 64 + lane) * EV * (int)sizeof(S);
    dst[i] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, POLICY));
  }
}

constexpr int kNonTemporal = 2;  // cache policy of the row streams (each row is read once)

// WPR = 8 (512 threads, 32 vectors per lane, softmax only): one row of up
// to 16384 vectors per CU, still a single pass; two waves per SIMD leave
// 256 VGPRs (the norms would also hold gamma / beta vectors per lane, and
// 16 waves of 16 vectors spilled at the 128 VGPRs four waves leave).
template <int OP, int DT, int WPR, int VPL>
__global__ void __launch_bounds__(WPR > 4 ? 64 * WPR : 256) row_vec_kernel(RowArgs a) {
  typedef typename Elem<DT>::storage S;
  static_assert(WPR <= 4 || OP == ROW_SOFTMAX, "8-wave rows: softmax only");
  // one reduction buffer per exchange (a row takes at most two), so no
  // exchange waits for the readers of a previous one
  constexpr int NRED = WPR > 4 ? WPR : 4;
  __shared__ float red[2 * NRED];

  const int lane = threadIdx.x & 63;
  // wave index and row as provably uniform values: the row's buffer
  // descriptors below are built from them and must live in scalar registers
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int rows_per_block = WPR >= 4 ? 1 : 4 / WPR;
  const int wave_in_row = (WPR == 1) ? 0 : wave;
  const int64_t row = (int64_t)blockIdx.x * rows_per_block + (WPR == 1 ? wave : 0);
  if (row >= a.rows) return;
  const int row_bytes = (int)(a.cols * (int64_t)sizeof(S));

  // Gamma / beta are fetched with the row, so their latency hides under the
  // row's own loads rather than stalling the write-back after the reduction.
  v4u raw[VPL], wv[VPL], bv[VPL];
  row_vec_load<DT, WPR, VPL, kNonTemporal>(a.x, a.ldx, row, row_bytes, wave_in_row, lane, raw);
#pragma unroll
  for (int i = 0; i < VPL; ++i) wv[i] = bv[i] = v4u{0u, 0u, 0u, 0u};
  if constexpr (OP != ROW_SOFTMAX)
    row_vec_load<DT, WPR, VPL, 0>(a.w, 0, 0, a.w ? row_bytes : 0, wave_in_row, lane, wv);
  if constexpr (OP == ROW_LAYERNORM)
    row_vec_load<DT, WPR, VPL, 0>(a.b, 0, 0, a.b ? row_bytes : 0, wave_in_row, lane, bv);
  row_vec_finish<OP, DT, WPR, VPL, NRED>(a, row, wave, lane, raw, wv, bv, red);
}

// Streaming form of the four-wave rows: a grid of G workgroups (a few per
// CU) walks the rows with stride G.  Gamma / beta are loaded once per
// workgroup and stay in registers, and each row's loads are issued before
// the previous row's reduction, so every workgroup keeps two rows in flight
// instead of one row per short-lived workgroup.  The two row buffers
// alternate without copies (a register copy would wait for the prefetch),
// and so do the two LDS exchange buffers: a wave writes buffer p for row
// k + 2 only after the barrier of row k + 1, which every wave reaches after
// reading buffer p for row k.
template <int OP, int DT, int VPL>
__global__ void __launch_bounds__(256) row_stream_kernel(RowArgs a) {
  typedef typename Elem<DT>::storage S;
  constexpr int WPR = 4, NRED = 4;
  __shared__ float red[2][2 * NRED];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int row_bytes = (int)(a.cols * (int64_t)sizeof(S));
  const int64_t stride = gridDim.x;
  int64_t row = blockIdx.x;  // the grid is no larger than the row count

  v4u b0[VPL], b1[VPL], wv[VPL], bv[VPL];
  row_vec_load<DT, WPR, VPL, kNonTemporal>(a.x, a.ldx, row, row_bytes, wave, lane, b0);
#pragma unroll
  for (int i = 0; i < VPL; ++i) wv[i] = bv[i] = v4u{0u, 0u, 0u, 0u};
  if constexpr (OP != ROW_SOFTMAX)
    row_vec_load<DT, WPR, VPL, 0>(a.w, 0, 0, a.w ? row_bytes : 0, wave, lane, wv);
  if constexpr (OP == ROW_LAYERNORM)
    row_vec_load<DT, WPR, VPL, 0>(a.b, 0, 0, a.b ? row_bytes : 0, wave, lane, bv);
  for (;;) {
    int64_t next = row + stride;
    row_vec_load<DT, WPR, VPL, kNonTemporal>(a.x, a.ldx, next < a.rows ? next : 0,
                                             next < a.rows ? row_bytes : 0, wave, lane, b1);
    row_vec_finish<OP, DT, WPR, VPL, NRED>(a, row, wave, lane, b0, wv, bv, red[0]);
    if (next >= a.rows) break;
    row = next;
    next = row + stride;
    row_vec_load<DT, WPR, VPL, kNonTemporal>(a.x, a.ldx, next < a.rows ? next : 0,
                                             next < a.rows ? row_bytes : 0, wave, lane, b0);
    row_vec_finish<OP, DT, WPR, VPL, NRED>(a, row, wave, lane, b1, wv, bv, red[1]);
    if (next >= a.rows) break;
    row = next;
  }
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
// Row configurations.  The streaming form keeps gamma / beta resident and
// two rows in flight per workgroup; measured on MI355X (8192 x 4096 f16,
// one process, interleaved): RMSNorm 24.6 -> 23.7 us and LayerNorm
// 27.6 -> 25.3 us with 4 workgroups per CU, while softmax (no gamma) is
// faster with one short-lived workgroup per row (23.6 against 24.4 us).
struct RowConfig {
  const char* name;
  int per_cu;  // workgroups per CU of the streaming form; 0: one row per workgroup
};
static const RowConfig kRowConfigs[] = {{"row", 0}, {"stream_2", 2}, {"stream_4", 4}, {"stream_8", 8}};
constexpr int kRowConfigCount = (int)(sizeof(kRowConfigs) / sizeof(kRowConfigs[0]));

int row_config_count() { return kRowConfigCount; }
const char* row_config_name(int cfg) { return cfg >= 0 && cfg < kRowConfigCount ? kRowConfigs[cfg].name : nullptr; }
int row_config_per_cu(int cfg) { return cfg >= 0 && cfg < kRowConfigCount ? kRowConfigs[cfg].per_cu : 0; }

// 16-byte vectors per row that the streaming form takes (four waves per row,
// 2 to 16 vectors per lane).
static bool row_stream_fits(int64_t vecs) { return vecs > 64 * 4 && vecs <= 256 * 16; }

int row_default_config(int op, int dtype, int64_t rows, int64_t cols) {
  if (op == ROW_OP_SOFTMAX) return 0;
  const int esize = dtype == DT_F32 ? 4 : 2;
  const int64_t vecs = (cols * esize + 15) / 16;
  if (!row_stream_fits(vecs)) return 0;
  // 4 workgroups per CU at 2 vectors per lane, 2 from 4 vectors up (more
  // registers per wave), and only with at least two rows per workgroup
  const int cfg = vecs <= 512 ? 2 : 1;
  return rows >= 2 * (int64_t)gemm_num_cus() * kRowConfigs[cfg].per_cu ? cfg : 0;
}

template <int OP, int DT, bool VEC>
static int launch_row_cfg(const RowArgs& a, hipStream_t s, int cfg) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  const int64_t vecs = (a.cols + EV - 1) / EV;  // 16-byte vectors per row
  const dim3 block(256);
  const int64_t g1 = (a.rows + 3) / 4;
  if constexpr (VEC) {
    // Short rows: one wave per row.  From 512 vectors (8 KiB) up, four waves
    // share a row with few vectors each, which keeps every wave small enough
    // for eight waves per SIMD (measured faster on MI355X than one wave
    // holding the whole row).
    const int per_cu = row_config_per_cu(cfg);
    if (per_cu > 0 && row_stream_fits(vecs)) {
      const int64_t gs = (int64_t)gemm_num_cus() * per_cu;
      const dim3 grid((unsigned)(gs < a.rows ? gs : a.rows));
      if (vecs <= 256 * 2) row_stream_kernel<OP, DT, 2><<<grid, block, 0, s>>>(a);
      else if (vecs <= 256 * 4) row_stream_kernel<OP, DT, 4><<<grid, block, 0, s>>>(a);
      else if (vecs <= 256 * 8) row_stream_kernel<OP, DT, 8><<<grid, block, 0, s>>>(a);
      else row_stream_kernel<OP, DT, 16><<<grid, block, 0, s>>>(a);
      return 0;
    }
    if (vecs <= 64 * 1) { row_vec_kernel<OP, DT, 1, 1><<<dim3(g1), block, 0, s>>>(a); }
    else if (vecs <= 64 * 4) { row_vec_kernel<OP, DT, 1, 4><<<dim3(g1), block, 0, s>>>(a); }
    else if (vecs <= 256 * 2) { row_vec_kernel<OP, DT, 4, 2><<<dim3(a.rows), block, 0, s>>>(a); }
    else if (vecs <= 256 * 4) { row_vec_kernel<OP, DT, 4, 4><<<dim3(a.rows), block, 0, s>>>(a); }
    else if (vecs <= 256 * 8) { row_vec_kernel<OP, DT, 4, 8><<<dim3(a.rows), block, 0, s>>>(a); }
    else if (vecs <= 256 * 16) { row_vec_kernel<OP, DT, 4, 16><<<dim3(a.rows), block, 0, s>>>(a); }
    else if constexpr (OP == ROW_SOFTMAX) {
      // one workgroup per row: with fewer than 64 rows most CUs would idle,
      // and the segmented two passes win (32 x 128256 f16: 19.6 against
      // 14.9 us; 64 x 32776: 10.2 against 13.9)
      if (vecs <= 512 * 32 && a.rows >= 64) row_vec_kernel<OP, DT, 8, 32><<<dim3(a.rows), dim3(512), 0, s>>>(a);
      else return HXI_ERR_UNSUPPORTED;
    } else return HXI_ERR_UNSUPPORTED;
  } else {
    if (vecs <= 64 * 1) { row_kernel<OP, DT, 1, 1, false><<<dim3(g1), block, 0, s>>>(a); }
    else if (vecs <= 64 * 4) { row_kernel<OP, DT, 1, 4, false><<<dim3(g1), block, 0, s>>>(a); }
    else if (vecs <= 64 * 8) { row_kernel<OP, DT, 1, 8, false><<<dim3(g1), block, 0, s>>>(a); }
    else if (vecs <= 256 * 8) { row_kernel<OP, DT, 4, 8, false><<<dim3(a.rows), block, 0, s>>>(a); }
    else if (vecs <= 256 * 16) { row_kernel<OP, DT, 4, 16, false><<<dim3(a.rows), block, 0, s>>>(a); }
    else return HXI_ERR_UNSUPPORTED;
  }
  return 0;
}

template <int OP, int DT>
static int launch_row_dt(const RowArgs& a, hipStream_t s, int cfg) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  bool vec = (a.cols % EV) == 0 && al16(a.x) && al16(a.y) &&
             ((a.ldx * (int64_t)sizeof(S)) % 16) == 0 && ((a.ldy * (int64_t)sizeof(S)) % 16) == 0 &&
             (a.w == nullptr || al16(a.w)) && (a.b == nullptr || al16(a.b));
  return vec ? launch_row_cfg<OP, DT, true>(a, s, cfg) : launch_row_cfg<OP, DT, false>(a, s, cfg);
}

template <int OP>
static int launch_row_op(int dtype, const RowArgs& a, hipStream_t s, int cfg) {
  if (cfg >= kRowConfigCount) return HXI_ERR_ARG;
  if (cfg < 0) cfg = row_default_config(OP, dtype, a.rows, a.cols);
  switch (dtype) {
    case DT_F16: return launch_row_dt<OP, DT_F16>(a, s, cfg);
    case DT_BF16: return launch_row_dt<OP, DT_BF16>(a, s, cfg);
    case DT_F32: return launch_row_dt<OP, DT_F32>(a, s, cfg);
    default: return HXI_ERR_DTYPE;
  }
}

int launch_softmax(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy,
                   int64_t rows, int64_t cols, hipStream_t s, int cfg) {
  RowArgs a{x, ldx, y, ldy, nullptr, nullptr, nullptr, nullptr, 0.f, rows, cols};
  return launch_row_op<ROW_SOFTMAX>(dtype, a, s, cfg);
}

int launch_rmsnorm(int dtype, const void* x, int64_t ldx, const void* gamma, float eps,
                   void* y, int64_t ldy, int64_t rows, int64_t cols, hipStream_t s, int cfg) {
  RowArgs a{x, ldx, y, ldy, gamma, nullptr, nullptr, nullptr, eps, rows, cols};
  return launch_row_op<ROW_RMSNORM>(dtype, a, s, cfg);
}

int launch_layernorm(int dtype, const void* x, int64_t ldx, const void* w, const void* b,
                     float eps, void* y, int64_t ldy, float* mean, float* rstd,
                     int64_t rows, int64_t cols, hipStream_t s, int cfg) {
  RowArgs a{x, ldx, y, ldy, w, b, mean, rstd, eps, rows, cols};
  return launch_row_op<ROW_LAYERNORM>(dtype, a, s, cfg);
}

// ---------------------------------------------------------------------------
// Rows longer than the register path holds (more than 4096 16-byte vectors):
// two passes over the row, the two-phase form of the reference's online
// softmax (test/python/triton/test_online_softmax.py:28-78; Milakov and
// Gimelshein, "Online normalizer calculation for softmax", 2018) applied to
// all three ops.  Each row is cut into S segments of L elements (L a
// multiple of one 256-thread sweep); workgroup b handles segment b % S of
// row b / S.
//   pass 1 (row_long_stats_kernel) folds its segment into one statistic:
//     softmax   (m, l): the maximum, and the sum of exp(x - m);
//     RMSNorm   the sum of x^2;
//     LayerNorm (n, mean, M2), merged with Chan, Golub and LeVeque's
//               pairwise update (mean += d n2 / n, M2 += M2' + d^2 n1 n2 / n);
//   pass 2 (row_long_apply_kernel) merges the row's S statistics and writes
//   its segment as the register path would with the merged values.  It walks
//   the workgroups in reverse, so the rows pass 1 read last are read again
//   first, while the 256 MB MALL still holds them.
// Every merge runs in a fixed order (lower index first), so results do not
// depend on scheduling.  The row is read twice and written once; each thread
// has kLongUnroll 16-byte loads in flight.
struct RowStat { float a, b, c, d; };

template <int OP>
__device__ __forceinline__ RowStat stat_identity() {
  if constexpr (OP == ROW_SOFTMAX) return RowStat{-INFINITY, 0.f, 0.f, 0.f};
  else return RowStat{0.f, 0.f, 0.f, 0.f};
}

template <int OP>
__device__ __forceinline__ RowStat stat_merge(RowStat x, RowStat y) {
  if constexpr (OP == ROW_SOFTMAX) {
    const float m = fmaxf(x.a, y.a);
    if (m == -INFINITY) return x;  // nothing but -inf so far: l stays 0
    return RowStat{m, x.b * fast_exp(x.a - m) + y.b * fast_exp(y.a - m), 0.f, 0.f};
  } else if constexpr (OP == ROW_RMSNORM) {
    return RowStat{x.a + y.a, 0.f, 0.f, 0.f};
  } else {
    // (a, b, c) = (n, mean, M2)
    const float n = x.a + y.a;
    if (n == 0.f) return x;
    const float d = y.b - x.b;
    const float f = y.a / n;
    return RowStat{n, x.b + d * f, x.c + y.c + d * d * x.a * f, 0.f};
  }
}

// Merge lane 0..63's statistics into lane 0 (lower lane first at each step).
template <int OP>
__device__ __forceinline__ RowStat stat_wave_reduce(RowStat v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    RowStat u{__shfl_down(v.a, o, 64), __shfl_down(v.b, o, 64), __shfl_down(v.c, o, 64), 0.f};
    if ((threadIdx.x & 63) + o < 64) v = stat_merge<OP>(v, u);
  }
  return v;
}

// The statistic of `cnt` consecutive elements held by one thread.
template <int OP, int EV>
__device__ __forceinline__ RowStat stat_of(const float* v, int cnt) {
  if constexpr (OP == ROW_SOFTMAX) {
    float m = -INFINITY;
    for (int j = 0; j < cnt; ++j) m = fmaxf(m, v[j]);
    if (m == -INFINITY) return RowStat{m, 0.f, 0.f, 0.f};
    float l = 0.f;
    for (int j = 0; j < cnt; ++j) l += fast_exp(v[j] - m);
    return RowStat{m, l, 0.f, 0.f};
  } else if constexpr (OP == ROW_RMSNORM) {
    float ss = 0.f;
    for (int j = 0; j < cnt; ++j) ss += v[j] * v[j];
    return RowStat{ss, 0.f, 0.f, 0.f};
  } else {
    if (cnt == 0) return RowStat{0.f, 0.f, 0.f, 0.f};
    float s = 0.f;
    for (int j = 0; j < cnt; ++j) s += v[j];
    const float mean = s / (float)cnt;
    float m2 = 0.f;
    for (int j = 0; j < cnt; ++j) m2 += (v[j] - mean) * (v[j] - mean);
    return RowStat{(float)cnt, mean, m2, 0.f};
  }
}

// Load the EV elements of vector `vi` of the row (columns vi*EV ..), those
// at or past `cols` reading as absent (the count is returned).
template <int DT, bool VEC>
__device__ __forceinline__ int load_vec(const typename Elem<DT>::storage* xr, int64_t vi, int64_t cols,
                                        float* v) {
  typedef typename Elem<DT>::storage S;
  constexpr int EV = 16 / sizeof(S);
  const int64_t c0 = vi * EV;
  if (c0 >= cols) return 0;
  if constexpr (VEC) {
    const v4u raw = *reinterpret_cast<const v4u*>(xr + c0);
    const S* e = reinterpret_cast<const S*>(&raw);
#pragma unroll
    for (int j = 0; j < EV; ++j) v[j] = Elem<DT>::load(e[j]);
    return EV;
  } else {
    const int cnt = (int)min((int64_t)EV, cols - c0);
    for (int j = 0; j < cnt; ++j) v[j] = Elem<DT>::load(xr[c0 + j]);
    return cnt;
  }
}

constexpr int kLongUnroll = 4;

template <int OP, int DT, bool VEC>
__global__ void __launch_bounds__(256) row_long_stats_kernel(RowArgs a, int S, int64_t seg_vecs, RowStat* st) {
  typedef typename Elem<DT>::storage Sx;
  constexpr int EV = 16 / sizeof(Sx);
  __shared__ RowStat red[4];
  const int64_t row = blockIdx.x / S;
  const int seg = (int)(blockIdx.x - row * S);
  const Sx* xr = reinterpret_cast<const Sx*>(a.x) + row * a.ldx;
  const int64_t v0 = (int64_t)seg * seg_vecs;
  RowStat acc = stat_identity<OP>();
  for (int64_t i0 = threadIdx.x; i0 < seg_vecs; i0 += 256 * kLongUnroll) {
    float v[kLongUnroll][EV];
    int cnt[kLongUnroll];
#pragma unroll
    for (int u = 0; u < kLongUnroll; ++u) {
      const int64_t i = i0 + 256 * u;
      cnt[u] = i < seg_vecs ? load_vec<DT, VEC>(xr, v0 + i, a.cols, v[u]) : 0;
    }
#pragma unroll
    for (int u = 0; u < kLongUnroll; ++u) acc = stat_merge<OP>(acc, stat_of<OP, EV>(v[u], cnt[u]));
  }
  acc = stat_wave_reduce<OP>(acc);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    RowStat t = red[0];
#pragma unroll
    for (int w = 1; w < 4; ++w) t = stat_merge<OP>(t, red[w]);
    st[blockIdx.x] = t;
  }
}

template <int OP, int DT, bool VEC>
__global__ void __launch_bounds__(256) row_long_apply_kernel(RowArgs a, int S, int64_t seg_vecs, const RowStat* st) {
  typedef typename Elem<DT>::storage Sx;
  constexpr int EV = 16 / sizeof(Sx);
  __shared__ RowStat row_stat;
  const int64_t b = (int64_t)gridDim.x - 1 - blockIdx.x;  // reverse of pass 1's order
  const int64_t row = b / S;
  const int seg = (int)(b - row * S);
  // the row's S <= 64 statistics, merged by the first wave in segment order
  if (threadIdx.x < 64) {
    RowStat t = (int)threadIdx.x < S ? st[row * S + threadIdx.x] : stat_identity<OP>();
    t = stat_wave_reduce<OP>(t);
    if (threadIdx.x == 0) row_stat = t;
  }
  __syncthreads();
  const RowStat rs = row_stat;
  float scale, shift = 0.f;
  if constexpr (OP == ROW_SOFTMAX) {
    scale = 1.0f / rs.b;  // DivToMul: one reciprocal, then multiplies
    shift = rs.a;
  } else if constexpr (OP == ROW_RMSNORM) {
    scale = 1.0f / sqrtf(rs.a / (float)a.cols + a.eps);
  } else {
    scale = 1.0f / sqrtf(rs.c / (float)a.cols + a.eps);
    shift = rs.b;
    if (seg == 0 && threadIdx.x == 0) {
      if (a.mean) a.mean[row] = rs.b;
      if (a.rstd) a.rstd[row] = scale;
    }
  }
  const Sx* xr = reinterpret_cast<const Sx*>(a.x) + row * a.ldx;
  Sx* yr = reinterpret_cast<Sx*>(a.y) + row * a.ldy;
  const Sx* wp = reinterpret_cast<const Sx*>(a.w);
  const Sx* bp = reinterpret_cast<const Sx*>(a.b);
  const int64_t v0 = (int64_t)seg * seg_vecs;
  for (int64_t i0 = threadIdx.x; i0 < seg_vecs; i0 += 256 * kLongUnroll) {
    float v[kLongUnroll][EV];
    int cnt[kLongUnroll];
#pragma unroll
    for (int u = 0; u < kLongUnroll; ++u) {
      const int64_t i = i0 + 256 * u;
      cnt[u] = i < seg_vecs ? load_vec<DT, VEC>(xr, v0 + i, a.cols, v[u]) : 0;
    }
#pragma unroll
    for (int u = 0; u < kLongUnroll; ++u) {
      const int64_t c0 = (v0 + i0 + 256 * u) * EV;
      Sx out[EV];
#pragma unroll
      for (int j = 0; j < EV; ++j) {
        if (j >= cnt[u]) break;
        float r;
        if constexpr (OP == ROW_SOFTMAX) {
          r = fast_exp(v[u][j] - shift) * scale;
        } else if constexpr (OP == ROW_RMSNORM) {
          r = v[u][j] * scale;
          if (wp) r = r * Elem<DT>::load(wp[c0 + j]);
        } else {
          r = (v[u][j] - shift) * scale;
          if (wp) r = r * Elem<DT>::load(wp[c0 + j]);
          if (bp) r = r + Elem<DT>::load(bp[c0 + j]);
        }
        out[j] = Elem<DT>::store(r);
      }
      if (VEC && cnt[u] == EV) {
        __builtin_nontemporal_store(*reinterpret_cast<const v4u*>(out), reinterpret_cast<v4u*>(yr + c0));
      } else {
        for (int j = 0; j < cnt[u]; ++j) yr[c0 + j] = out[j];
      }
    }
  }
}

// Segments: about 1024 workgroups over all rows, at most 64 per row, each
// at least four vectors per thread.
static void row_long_plan(int64_t rows, int64_t cols, int ev, int* S, int64_t* seg_vecs) {
  const int64_t vecs = (cols + ev - 1) / ev;
  int64_t s = std::min<int64_t>((1024 + rows - 1) / rows, 64);
  s = std::max<int64_t>(1, std::min<int64_t>(s, vecs / (256 * 4)));
  int64_t sv = (vecs + s - 1) / s;
  sv = (sv + 255) / 256 * 256;
  *seg_vecs = sv;
  *S = (int)((vecs + sv - 1) / sv);
}

size_t row_long_ws_bytes(int dtype, int64_t rows, int64_t cols) {
  int S;
  int64_t sv;
  row_long_plan(rows, cols, dtype == DT_F32 ? 4 : 8, &S, &sv);
  return (size_t)rows * S * sizeof(RowStat);
}

template <int OP, int DT, bool VEC>
static int launch_row_long_cfg(const RowArgs& a, void* ws, hipStream_t s) {
  constexpr int EV = DT == DT_F32 ? 4 : 8;
  int S;
  int64_t sv;
  row_long_plan(a.rows, a.cols, EV, &S, &sv);
  const int64_t blocks = a.rows * S;
  if (blocks >= ((int64_t)1 << 31)) return HXI_ERR_SHAPE;
  RowStat* st = static_cast<RowStat*>(ws);
  row_long_stats_kernel<OP, DT, VEC><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a, S, sv, st);
  row_long_apply_kernel<OP, DT, VEC><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(a, S, sv, st);
  return 0;
}

template <int OP, int DT>
static int launch_row_long_dt(const RowArgs& a, void* ws, hipStream_t s) {
  typedef typename Elem<DT>::storage Sx;
  constexpr int EV = 16 / sizeof(Sx);
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool vec = (a.cols % EV) == 0 && al16(a.x) && al16(a.y) &&
                   ((a.ldx * (int64_t)sizeof(Sx)) % 16) == 0 && ((a.ldy * (int64_t)sizeof(Sx)) % 16) == 0;
  return vec ? launch_row_long_cfg<OP, DT, true>(a, ws, s) : launch_row_long_cfg<OP, DT, false>(a, ws, s);
}

int launch_row_long(int op, int dtype, const void* x, int64_t ldx, const void* w, const void* b, float eps,
                    void* y, int64_t ldy, float* mean, float* rstd, int64_t rows, int64_t cols, void* ws,
                    hipStream_t s) {
  RowArgs a{x, ldx, y, ldy, w, b, mean, rstd, eps, rows, cols};
  auto by_dt = [&](auto opc) -> int {
    constexpr int OP = decltype(opc)::value;
    switch (dtype) {
      case DT_F16: return launch_row_long_dt<OP, DT_F16>(a, ws, s);
      case DT_BF16: return launch_row_long_dt<OP, DT_BF16>(a, ws, s);
      case DT_F32: return launch_row_long_dt<OP, DT_F32>(a, ws, s);
      default: return HXI_ERR_DTYPE;
    }
  };
  switch (op) {
    case ROW_SOFTMAX: return by_dt(std::integral_constant<int, ROW_SOFTMAX>{});
    case ROW_RMSNORM: return by_dt(std::integral_constant<int, ROW_RMSNORM>{});
    case ROW_LAYERNORM: return by_dt(std::integral_constant<int, ROW_LAYERNORM>{});
    default: return HXI_ERR_ARG;
  }
}

// ---------------------------------------------------------------------------
// SiLU * mul: out = RNE(silu(g) * u), silu(g) = g / (1 + exp(-g)).  fp16
// rows, 16-byte vectors; a grid-stride loop over 8-element groups.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256) silu_mul_f16_kernel(
    const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu, uint16_t* o, int64_t ldo,
    int64_t rows, int64_t cols) {
  const int64_t groups_per_row = cols / 8;
  const int64_t total = rows * groups_per_row;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / groups_per_row, c = (t - r * groups_per_row) * 8;
    const v4u gv = *reinterpret_cast<const v4u*>(g + r * ldg + c);
    const v4u uv = *reinterpret_cast<const v4u*>(u + r * ldu + c);
    const uint16_t* ge = reinterpret_cast<const uint16_t*>(&gv);
    const uint16_t* ue = reinterpret_cast<const uint16_t*>(&uv);
    uint16_t out[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = silu_mul_h(ge[j], ue[j]);
    *reinterpret_cast<v4u*>(o + r * ldo + c) = *reinterpret_cast<const v4u*>(out);
  }
}

__global__ void __launch_bounds__(256) silu_mul_f16_scalar_kernel(
    const uint16_t* g, int64_t ldg, const uint16_t* u, int64_t ldu, uint16_t* o, int64_t ldo,
    int64_t rows, int64_t cols) {
  const int64_t total = rows * cols;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = t / cols, c = t - r * cols;
    o[r * ldo + c] = silu_mul_h(g[r * ldg + c], u[r * ldu + c]);
  }
}

int launch_silu_mul_f16(const void* g, int64_t ldg, const void* u, int64_t ldu, void* o,
                        int64_t ldo, int64_t rows, int64_t cols, hipStream_t s) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const bool vec = cols % 8 == 0 && ldg % 8 == 0 && ldu % 8 == 0 && ldo % 8 == 0 && al16(g) &&
                   al16(u) && al16(o);
  const int64_t work = vec ? rows * (cols / 8) : rows * cols;
  int64_t blocks = (work + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  if (blocks < 1) blocks = 1;
  if (vec)
    silu_mul_f16_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (uint16_t*)o, ldo, rows, cols);
  else
    silu_mul_f16_scalar_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        (const uint16_t*)g, ldg, (const uint16_t*)u, ldu, (uint16_t*)o, ldo, rows, cols);
  return 0;
}

}  // namespace hx
