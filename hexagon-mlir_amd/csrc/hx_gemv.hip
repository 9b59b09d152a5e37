// hx_gemv.hip -- W8A16 decode GEMM/GEMV for M <= 16:
//   Y[m][n] = RNE_f16( (sum_k X[m][k] * W[k][n]) * s[n] ),  binary32 accumulate.
//
// In hexagon-mlir the M <= 4 rows are refused by the HMX engine as
// `min-rows` and M = 16 fails `tile-alignment` (QHB/include/hexagon/Dialect/
// Hmx/Transforms/HmxTarget.h:100, 195-218), so these shapes run through the
// HVX (i,k,j) generic of ScheduleMatmulForHVX
// (QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:169-196) with the
// dequantised weight (sitofp, then the per-channel scale).
//
// MI355X design: the kernel is an HBM stream over the int8 weight, read once,
// K-contiguous ([N][K], the resident image).  One wave owns 16*CT output
// columns and a slice of K; every 128-wide K window it loads, per column, 128
// contiguous weight bytes (two 16-byte loads per lane, each covering 64
// contiguous bytes of 16 rows), widens int8 -> f16 exactly in registers and
// feeds v_mfma_f32_16x16x32_f16 with the (zero-padded to 16 rows)
// activations.  Lane group g = lane/16 supplies k = 64*h + 16*g + 8*e + (0..7)
// in step s = 2h + e for both operands, so every k of the window is summed
// exactly once.  The four waves of a workgroup split K and reduce through
// LDS; with KS > 1 workgroups split K further and the last one to finish a
// column tile (atomic ticket) sums the KS partials in a fixed order, so the
// result is deterministic.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

__device__ __forceinline__ v4i gv_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int CT, int KS>
__global__ void __launch_bounds__(256) gemv_w8a16_kernel(GemvArgs p) {
  constexpr int UNR = 4;  // K windows loaded per batch
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int col_tile = blockIdx.x;
  const int ks = (KS > 1) ? blockIdx.y : 0;
  const int64_t n0 = (int64_t)col_tile * 16 * CT;
  const int64_t cols_valid = min((int64_t)16 * CT, p.N - n0);

  const uint32_t ldw = (uint32_t)p.ldw;
  const uint32_t ldx_b = (uint32_t)(p.ldx * 2);
  const uint32_t kbytes_x = (uint32_t)(p.K * 2);
  const uint32_t kbytes_w = (uint32_t)p.K;
  __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.w + n0 * p.ldw), 0, (int)(cols_valid * p.ldw), 0x00020000);
  __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.x, 0, (int)(p.M * ldx_b), 0x00020000);
  const bool xrow = nl < p.M;

  const int nwin = (int)((p.K + 127) / 128);
  const int per_split = (nwin + KS - 1) / KS;
  const int w_begin = ks * per_split;
  const int w_end = min(nwin, w_begin + per_split);

  v4f acc[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int wb = w_begin + wave; wb < w_end; wb += 4 * UNR) {
    v4i wq[UNR][CT][2];
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int win = wb + 4 * u;
#pragma unroll
      for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t kb = (uint32_t)win * 128u + 64u * h + 16u * g;
          const uint32_t off = (win < w_end && kb < kbytes_w)
                                   ? (uint32_t)(16 * c + nl) * ldw + kb : 0x80000000u;
          wq[u][c][h] = gv_load16(rw, off);
        }
    }
#pragma unroll
    for (int u = 0; u < UNR; ++u) {
      const int win = wb + 4 * u;
      v4i xq[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int h = s >> 1, e = s & 1;
        const uint32_t kx = ((uint32_t)win * 128u + 64u * h + 16u * g + 8u * e) * 2u;
        const uint32_t off = (xrow && win < w_end && kx < kbytes_x)
                                 ? (uint32_t)nl * ldx_b + kx : 0x80000000u;
        xq[s] = gv_load16(rx, off);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int h = s >> 1, e = s & 1;
        const v8h xa = __builtin_bit_cast(v8h, xq[s]);
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          const v8h wb16 = i8x8_to_v8h((uint32_t)wq[u][c][h][2 * e], (uint32_t)wq[u][c][h][2 * e + 1]);
          acc[c] = mfma16_f16(xa, wb16, acc[c]);
        }
      }
    }
  }

  // ---- reduce the four waves' partial tiles through LDS ----------------
  __shared__ float red[4][CT][64][4];
  __shared__ int is_last;
#pragma unroll
  for (int c = 0; c < CT; ++c)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][c][lane][r] = acc[c][r];
  __syncthreads();

  // Thread t finalises CT elements: (c, l, r) with l = t / 4, r = t % 4.
  const int fl = tid >> 2, fr = tid & 3;
  const int fm = 4 * (fl >> 4) + fr;           // output row (activation row)
  float sum[CT];
#pragma unroll
  for (int c = 0; c < CT; ++c)
    sum[c] = ((red[0][c][fl][fr] + red[1][c][fl][fr]) + red[2][c][fl][fr]) + red[3][c][fl][fr];

  uint16_t* y = reinterpret_cast<uint16_t*>(p.y);
  if constexpr (KS == 1) {
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int64_t n = n0 + 16 * c + (fl & 15);
      if (fm < p.M && n < p.N)
        y[(int64_t)fm * p.ldy + n] = f32_to_f16_bits(p.scale ? sum[c] * p.scale[n] : sum[c]);
    }
  } else {
    // partial[ks][m][n]
#pragma unroll
    for (int c = 0; c < CT; ++c) {
      const int64_t n = n0 + 16 * c + (fl & 15);
      if (fm < p.M && n < p.N) p.partial[((int64_t)ks * p.M + fm) * p.N + n] = sum[c];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
      const unsigned ticket = atomicAdd(&p.counters[col_tile], 1u);
      is_last = (ticket == (unsigned)(KS - 1));
    }
    __syncthreads();
    if (is_last) {
      __threadfence();
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        const int64_t n = n0 + 16 * c + (fl & 15);
        if (fm < p.M && n < p.N) {
          float t = 0.f;
          for (int s = 0; s < KS; ++s)
            t += __builtin_nontemporal_load(&p.partial[((int64_t)s * p.M + fm) * p.N + n]);
          y[(int64_t)fm * p.ldy + n] = f32_to_f16_bits(p.scale ? t * p.scale[n] : t);
        }
      }
      if (tid == 0) p.counters[col_tile] = 0u;  // ready for the next call
    }
  }
}

typedef void (*GemvLaunch)(const GemvArgs&, hipStream_t);

template <int CT, int KS>
static void gemv_launch_one(const GemvArgs& a, hipStream_t s) {
  const int64_t tiles = (a.N + 16 * CT - 1) / (16 * CT);
  gemv_w8a16_kernel<CT, KS><<<dim3((unsigned)tiles, KS), dim3(256), 0, s>>>(a);
}

struct GemvEntry {
  GemvConfig cfg;
  GemvLaunch fn;
};

static const GemvEntry kGemv[] = {
    {{1, 1, "ct1_ks1"}, &gemv_launch_one<1, 1>},
    {{2, 1, "ct2_ks1"}, &gemv_launch_one<2, 1>},
    {{1, 2, "ct1_ks2"}, &gemv_launch_one<1, 2>},
    {{2, 2, "ct2_ks2"}, &gemv_launch_one<2, 2>},
    {{4, 2, "ct4_ks2"}, &gemv_launch_one<4, 2>},
    {{4, 4, "ct4_ks4"}, &gemv_launch_one<4, 4>},
    {{2, 4, "ct2_ks4"}, &gemv_launch_one<2, 4>},
};

int gemv_config_count() { return (int)(sizeof(kGemv) / sizeof(kGemv[0])); }
const GemvConfig* gemv_config(int idx) {
  if (idx < 0 || idx >= gemv_config_count()) return nullptr;
  return &kGemv[idx].cfg;
}
int gemv_default_config(int64_t M, int64_t N, int64_t K) {
  (void)N; (void)K;
  return M <= 4 ? 0 : 3;
}
int64_t gemv_partial_floats(int cfg_idx, int64_t M, int64_t N) {
  const GemvConfig* c = gemv_config(cfg_idx);
  return (c && c->ks > 1) ? (int64_t)c->ks * M * N : 0;
}
int64_t gemv_counter_count(int cfg_idx, int64_t N) {
  const GemvConfig* c = gemv_config(cfg_idx);
  return (c && c->ks > 1) ? (N + 16 * c->ct - 1) / (16 * c->ct) : 0;
}
bool gemv_fast_ok(const GemvArgs& a) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.M < 1 || a.M > 16 || a.N < 1 || a.K < 1) return false;
  if (a.K % 16 != 0 || a.ldw % 16 != 0 || (a.ldx * 2) % 16 != 0) return false;
  if (!al16(a.x) || !al16(a.w)) return false;
  if ((int64_t)64 * a.ldw >= ((int64_t)1 << 31)) return false;
  if ((int64_t)a.M * a.ldx * 2 >= ((int64_t)1 << 31)) return false;
  return true;
}
int launch_gemv_w8a16(int cfg_idx, const GemvArgs& a, hipStream_t s) {
  if (cfg_idx < 0 || cfg_idx >= gemv_config_count()) return HXI_ERR_ARG;
  if (kGemv[cfg_idx].cfg.ks > 1 && (a.partial == nullptr || a.counters == nullptr)) return HXI_ERR_ARG;
  kGemv[cfg_idx].fn(a, s);
  return HXI_OK;
}

}  // namespace hx
