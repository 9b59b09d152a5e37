// hx_gemv.hip -- decode GEMM/GEMV for M <= 16, int8 (W8A16), f16 or bf16
// weights:
//   Y[m][n] = RNE( (sum_k X[m][k] * W[k][n]) * s[n] ),  binary32 accumulate,
// rounded to the activations' type.
//
// In hexagon-mlir the M <= 4 rows are refused by the HMX engine as
// `min-rows` and M = 16 fails `tile-alignment` (QHB/include/hexagon/Dialect/
// Hmx/Transforms/HmxTarget.h:100, 195-218), so these shapes run through the
// HVX (i,k,j) generic of ScheduleMatmulForHVX
// (QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:169-196), for int8 with
// the dequantised weight (sitofp, then the per-channel scale).
//
// MI355X design: an HBM stream over the weight, read once, fed to
// v_mfma_f32_16x16x32_{f16,bf16} with the activations zero-padded to 16
// rows (int8 widened to f16 exactly in registers).  Two kernels:
//   * gemv_stream_kernel -- registered int8 weights, stored in MFMA fragment
//     order so that every wave load is one contiguous KiB, and f16/bf16
//     weights read in place from [N][K]; each wave issues its K slice before
//     its first MFMA (below);
//   * gemv_w8a16_kernel -- an unregistered K-contiguous [N][K] int8 weight:
//     per 128-wide K window each lane loads 2 x 16 bytes of one column; lane
//     group g = lane/16 supplies k = 64*h + 16*g + 8*e + (0..7) in step
//     s = 2h + e for both operands, so every k is summed exactly once; the
//     four waves of a workgroup split K and reduce through LDS.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

// s * scale[n] in binary32 (an f16 scale is widened exactly), or s without
// a scale.
__device__ __forceinline__ float gv_scaled(const GemvArgs& p, int64_t n, float s) {
  if (p.scale) return s * p.scale[n];
  if (p.scale16) return s * f16_bits_to_f32(p.scale16[n]);
  return s;
}

// activation staging of the packed kernel: none (register fragments per
// chunk), LDS filled through registers, LDS filled by direct-to-LDS loads
enum GemvXStage : int { XS_NONE = 0, XS_REG = 1, XS_DMA = 2 };

__device__ __forceinline__ v4i gv_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int CT>
__global__ void __launch_bounds__(256) gemv_w8a16_kernel(GemvArgs p) {
  constexpr int UNR = 4;  // K windows loaded per batch
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int col_tile = blockIdx.x;
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

  const int w_begin = 0;
  const int w_end = (int)((p.K + 127) / 128);

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
#pragma unroll
  for (int c = 0; c < CT; ++c) {
    const int64_t n = n0 + 16 * c + (fl & 15);
    if (fm < p.M && n < p.N)
      y[(int64_t)fm * p.ldy + n] = f32_to_f16_bits(gv_scaled(p, n, sum[c]));
  }
}

// ---------------------------------------------------------------------------
// Streaming kernel for registered int8 weights (fragment-packed image) and
// for f16/bf16 weights read in place from a K-contiguous [N][K] matrix.
//
// A K chunk is the 1 KiB a wave loads per 16-column tile: 64 k of int8 or 32
// k of f16/bf16.  Lane l = 16g + c of the wave loads the 16 bytes of column
// c, k = KD*j + (KD/4)*g + (0..KD/4-1) of chunk j, which feed the
// v_mfma_f32_16x16x32 steps e (k = .. + 8e + (0..7)): two steps for int8
// (widened to f16 in registers), one for f16/bf16; the activation operand
// uses the same k mapping.
//   * int8, packed: for column tile t and chunk j one 1 KiB block at
//     ((t * KC) + j) * 1024 (KC chunks per tile), in which byte
//     256*g + 16*c + i holds W[64*j + 16*g + i][16*t + c] ^ 0x80 (g 0..3,
//     c 0..15, i 0..15; excess-128, so the widening needs no XOR per load),
//     so every wave load is one contiguous KiB;
//   * f16/bf16, packed (registered weights): block (t, j) at ((t * KC) + j)
//     * 1024, in which bytes 256*g + 16*c .. + 15 hold W[32*j + 8*g + (0..7)]
//     [16*t + c] (zero beyond N and K);
//   * f16/bf16, in place: lane l reads row 16t + c of the [N][K] weight at
//     k = 32j + 8g: sixteen 64-byte runs per wave load.  A pure read of
//     134 MB in that pattern takes 31 us against 21-22 us in contiguous
//     KiBs (N = K = 8192, 512 workgroups), which is what the packed image
//     buys.
// A workgroup of KW waves splits K into slices of CPW * KW chunks; each wave
// loads CPW chunks of each of its CT tiles per slice, ahead of the MFMAs
// that use them (how far ahead is the compiler's schedule: for the wide
// configs it interleaves loads and MFMAs with fewer live registers, which
// measured faster than holding the whole slice).  EAGER: a scheduling
// barrier keeps every load of the slice ahead of its first MFMA instead,
// which the narrower configs gain from.  With K = 4096 int8 and
// CPW * KW = 64 a slice is all of K.  PIPE: two register sets, the next
// slice's loads issued before the current slice's MFMAs.
//
// XL (M <= 4): the activations are staged once per workgroup in LDS ([M]
// rows of kchunks*KD, zero-padded), and each MFMA step reads its operand
// from there; the registers that would hold every step's activation
// fragment are freed, so more waves -- more weight bytes in flight -- fit
// on a CU.  The activation loads are issued before the weight stream: loads
// complete in issue order, so an activation load queued behind a wave's
// weight loads would hold back the whole workgroup's compute (the LDS
// staging ends in a barrier) until its last weight byte has arrived,
// leaving no overlap between compute and stream.
template <int WT>
__device__ __forceinline__ v4f gv_mfma(v4u a, v4u b, v4f c) {
  if constexpr (WT == DT_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c,
                                                    0, 0, 0);
  else
    return mfma16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c);
}

// MB > 1 (16 < M <= 16 MB): MB blocks of 16 activation rows; every weight
// fragment feeds MB MFMAs, so the weight is still streamed once.
template <int CT, int KW, int CPW, int XS, int WT, bool PK, bool PIPE, int MB = 1, bool SPLIT = false,
          bool EAGER = false>
__global__ void __launch_bounds__(64 * KW) gemv_stream_kernel(GemvArgs p, const void* wsrc, int64_t ldw,
                                                              int kchunks) {
  static_assert(MB == 1 || (XS == XS_NONE && !PIPE), "row blocks: register-fragment configs only");
  constexpr bool XL = XS != XS_NONE;
  constexpr int KD = WT == DT_I8 ? 64 : 32;  // k per chunk
  constexpr int KG = KD / 4;                  // k per lane group within a chunk
  constexpr int NE = WT == DT_I8 ? 2 : 1;     // MFMA steps per chunk
  constexpr int ES = WT == DT_I8 ? 1 : 2;     // weight element bytes
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15, g = lane >> 4;
  // K split (non-staged, non-pipelined configs): workgroup b is part
  // b % parts of column-tile group b / parts and reduces chunks [kc0, kc1)
  // (a compile-time variant: the unsplit configs keep their code as it was)
  const int parts = SPLIT ? p.parts : 1;
  const int part = (int)(blockIdx.x % (unsigned)parts), grp = (int)(blockIdx.x / (unsigned)parts);
  const int cpp = (kchunks + parts - 1) / parts;
  const int kc0 = part * cpp, kc1 = min(kchunks, kc0 + cpp);
  const int t0 = grp * CT;                           // first column tile
  const int ntiles = (int)((p.N + 15) / 16);
  const int tiles_here = min(CT, ntiles - t0);
  const int rows_here = (int)min((int64_t)16 * CT, p.N - (int64_t)16 * t0);
  const bool xrow = col < p.M;
  const uint16_t* x = reinterpret_cast<const uint16_t*>(p.x);
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int64_t kp = (int64_t)kchunks * KD;
  constexpr int NT = 64 * KW;                     // threads
  constexpr int NSC = (CT * 256 + NT - 1) / NT;  // outputs per row block this thread finalises

  // The column scales this thread applies at the end, loaded first: issued
  // after the reduction, the load of a cold scale line would add its whole
  // memory latency to every launch.  Thread t finalises element
  // e = t + NT * i of each row block, column (t0 + e / 256) * 16 + (e / 4) % 16
  // (the reduction below); with M <= 4 (one row block, rows in lanes 0..15)
  // thread t < 64 CT finalises column (t0 + t / 64) * 16 + (t / 4) % 16.
  // Out-of-range offsets read zero and are never used.
  const bool few_rows = MB == 1 && p.M <= 4;
  float sc[NSC];
  {
    const bool s32 = p.scale != nullptr;
    const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
        s32 ? (void*)p.scale : (void*)p.scale16, 0,
        (s32 || p.scale16) ? (int)(p.N * (s32 ? 4 : 2)) : 0, 0x00020000);
#pragma unroll
    for (int i = 0; i < NSC; ++i) {
      const int e = tid + NT * i;
      const int64_t n = few_rows ? (int64_t)(t0 + (tid >> 6)) * 16 + ((tid >> 2) & 15)
                                 : (int64_t)(t0 + (e >> 8)) * 16 + ((e >> 2) & 15);
      const bool in = (few_rows ? (i == 0 && tid < 64 * CT) : e < CT * 256) && n < p.N;
      if (s32) {
        sc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rsc, in ? (int)(n * 4) : (int)0x80000000, 0, 0));
      } else {
        const uint16_t h = __builtin_amdgcn_raw_buffer_load_b16(rsc, in ? (int)(n * 2) : (int)0x80000000, 0, 0);
        sc[i] = f16_bits_to_f32(h);
      }
    }
  }
  const bool has_scale = p.scale != nullptr || p.scale16 != nullptr;
  // The SwiGLU gate values of this thread's outputs (p.gate: the fused
  // epilogue), loaded up front for the same reason as the scales; the
  // (row, column) of each is the one the reduction below finalises.
  uint16_t gv[MB][NSC];
  if (p.gate) {
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.gate, 0, (int)(p.M * p.ldg * 2), 0x00020000);
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
      for (int i = 0; i < NSC; ++i) {
        const int e = tid + NT * i;
        int64_t m, n;
        bool in;
        if (few_rows) {
          m = tid & 3;
          n = (int64_t)(t0 + (tid >> 6)) * 16 + ((tid >> 2) & 15);
          in = i == 0 && tid < 64 * CT;
        } else {
          const int l = (e >> 2) & 63;
          m = 16 * b + 4 * (l >> 4) + (e & 3);
          n = (int64_t)(t0 + (e >> 8)) * 16 + (l & 15);
          in = e < CT * 256;
        }
        in = in && m < p.M && n < p.N;
        gv[b][i] = __builtin_amdgcn_raw_buffer_load_b16(rg, in ? (int)((m * p.ldg + n) * 2) : (int)0x80000000, 0, 0);
      }
  }

  // Every global load below is a buffer load whose out-of-range offset
  // (0x80000000) reads zero, so no load sits behind a branch: a conditional
  // load makes the compiler wait for it at the join, or count outstanding
  // loads conservatively.  The launcher keeps all offsets below 2^31.
  const char* wbase = reinterpret_cast<const char*>(wsrc) +
                      (PK ? (int64_t)t0 * kchunks * 1024 : (int64_t)16 * t0 * ldw * ES);
  const int wbytes = PK ? tiles_here * kchunks * 1024 : (int)((int64_t)rows_here * ldw * ES);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc((void*)wbase, 0, wbytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, (int)(p.M * p.ldx * 2), 0x00020000);
  constexpr int kNT = 2;  // cache policy: non-temporal (the weight is streamed once)

  v4f acc[MB][CT];
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int c = 0; c < CT; ++c) acc[b][c] = v4f{0.f, 0.f, 0.f, 0.f};

  // XL staging of the [M][kp] activation block into LDS, issued ahead of the
  // weight stream.  Rows are XLP elements apart (kp rounded up to whole
  // 1 KiB blocks, plus 8: a block never spills into the next row, and the
  // 16-byte skew spreads the rows over the LDS banks); elements at or past K
  // read zero.
  //   XS_DMA: direct-to-LDS loads (no registers held, no copy); 1 KiB block
  //     b = (row m, 512-element segment j) is loaded by wave b % KW.
  //   XS_REG: the block is walked as (row m, column block b): step
  //     r = m * cb + b covers the 16-byte chunks b * T + tid of row m (T
  //     threads, cb blocks per row); the first XR steps go through registers
  //     ahead of the weight loads, any further ones are loaded after them.
  // Measured at N = 11008, K = 4096 (int8): DMA is faster for M = 1 (one
  // load per wave), registers for M = 4 (the DMA's LDS writes delay the
  // weight loads queued behind them).
  const int bpr = (int)((kp + 511) / 512);  // 1 KiB blocks per row
  const int64_t xlp = (int64_t)bpr * 512 + 8;
  constexpr int XR = XS == XS_REG ? (2048 / NT > 0 ? 2048 / NT : 1) : 1;
  const uint32_t row_ch = (uint32_t)(kp / 8);
  const uint32_t cb = (row_ch + NT - 1) / NT;
  const uint32_t nsteps = XS == XS_REG ? (uint32_t)p.M * cb : 0u;
  auto x_load = [&](uint32_t r) -> v4u {  // step r; zero past K or past the last step
    const uint32_t m = r / cb, k = ((r - m * cb) * NT + (uint32_t)tid) * 8u;
    const uint32_t off = (r < nsteps && k < (uint32_t)p.K) ? (m * (uint32_t)p.ldx + k) * 2u : 0x80000000u;
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
  };
  auto x_store = [&](uint32_t r, const v4u& v) {  // step r into xs (chunks past kp skipped)
    const uint32_t m = r / cb, c = (r - m * cb) * NT + (uint32_t)tid;
    if (c < row_ch) *reinterpret_cast<v4u*>(xs + (int64_t)m * xlp + c * 8u) = v;
  };
  v4u xr[XR];
  if constexpr (XS == XS_REG) {
#pragma unroll
    for (int r = 0; r < XR; ++r) xr[r] = x_load((uint32_t)r);
  } else if constexpr (XS == XS_DMA) {
    const int nblk = (int)p.M * bpr;
    for (int blk = wave; blk < nblk; blk += KW) {
      const int m = blk / bpr, j = blk - m * bpr;
      const uint32_t k = (uint32_t)j * 512u + 8u * (uint32_t)lane;
      const uint32_t off = k < (uint32_t)p.K ? ((uint32_t)m * (uint32_t)p.ldx + k) * 2u : 0x80000000u;
      dma16(rx, reinterpret_cast<char*>(xs + (int64_t)m * xlp + (int64_t)j * 512), off, 0u);
    }
  }

  // chunks [c0, c0 + CPW * KW) are split as wave w -> c0 + w + KW * u
  constexpr int STEP = CPW * KW;
  // issue / compute of one K slice, for the pipelined path
  typedef v4u WFrag[CPW][CT];
  typedef v4u XFrag[XL ? 1 : CPW][NE];
  auto issue = [&](int c0, WFrag& wq, XFrag& xq) {
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int j = c0 + wave + KW * u;
      const bool jv = j < kchunks;
#pragma unroll
      for (int c = 0; c < CT; ++c) {
        uint32_t off;
        if constexpr (PK) {
          off = (jv && c < tiles_here) ? (uint32_t)(c * kchunks + j) * 1024u + 16u * (uint32_t)lane : 0x80000000u;
        } else {
          const uint32_t row = (uint32_t)(16 * c + col), k = (uint32_t)j * KD + KG * (uint32_t)g;
          off = (jv && row < (uint32_t)rows_here && k < (uint32_t)p.K)
                    ? (row * (uint32_t)ldw + k) * (uint32_t)ES : 0x80000000u;
        }
        wq[u][c] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, kNT));
      }
      if constexpr (!XL) {
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          const uint32_t k = (uint32_t)j * KD + KG * (uint32_t)g + 8u * e;
          const uint32_t off = (jv && xrow && k < (uint32_t)p.K)
                                   ? ((uint32_t)col * (uint32_t)p.ldx + k) * 2u : 0x80000000u;
          xq[u][e] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
        }
      }
    }
  };
  // XL: publish the staged activations.  XS_DMA: they have landed once no
  // more than the `after` weight loads issued behind them are outstanding
  // (loads complete in order); the LDS-only barrier does not wait for the
  // weight loads still in flight, as __syncthreads would.  XS_REG: copy
  // them in, then barrier.
  auto publish = [&](auto after) {
    if constexpr (XS == XS_REG) {
#pragma unroll
      for (int r = 0; r < XR; ++r)
        if ((uint32_t)r < nsteps) x_store((uint32_t)r, xr[r]);
      for (uint32_t r = XR; r < nsteps; ++r) x_store(r, x_load(r));
      __syncthreads();
    } else if constexpr (XS == XS_DMA) {
      wait_vm<decltype(after)::value>();
      lds_barrier();
    }
  };
  auto compute = [&](int c0, const WFrag& wq, const XFrag& xq) {
#pragma unroll
    for (int u = 0; u < CPW; ++u)
#pragma unroll
      for (int e = 0; e < NE; ++e) {
        v4u xa;
        if constexpr (XL) {
          // only the lanes of rows < M read (the others hold zeros): with
          // M = 1 a read moves 4 lanes' bytes instead of 64
          const int64_t k = (int64_t)(c0 + wave + KW * u) * KD + KG * g + 8 * e;
          xa = v4u{0u, 0u, 0u, 0u};
          if (xrow && k < kp) xa = *reinterpret_cast<const v4u*>(xs + col * xlp + k);
        } else {
          xa = xq[u][e];
        }
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          v4u wb;
          if constexpr (WT == DT_I8)
            wb = __builtin_bit_cast(v4u, PK ? x8x8_to_v8h(wq[u][c][2 * e], wq[u][c][2 * e + 1])
                                         : i8x8_to_v8h(wq[u][c][2 * e], wq[u][c][2 * e + 1]));
          else
            wb = wq[u][c];
          acc[0][c] = gv_mfma<WT>(xa, wb, acc[0][c]);
        }
      }
  };

  if constexpr (!PIPE) {
    // Each K slice of STEP chunks is one round trip: issue, then compute.
    // Written out here rather than through issue/compute: the compiler then
    // schedules the slice's loads among its MFMAs with fewer live registers,
    // which measured up to 2x faster for the wide (CT >= 2, CPW = 8) configs.
    for (int c0 = kc0; c0 < kc1; c0 += STEP) {
      v4u wq[CPW][CT];
      v4u xq[XL ? 1 : CPW][NE][MB];
#pragma unroll
      for (int u = 0; u < CPW; ++u) {
        const int j = c0 + wave + KW * u;
        const bool jv = j < kc1;
#pragma unroll
        for (int c = 0; c < CT; ++c) {
          uint32_t off;
          if constexpr (PK) {
            off = (jv && c < tiles_here) ? (uint32_t)(c * kchunks + j) * 1024u + 16u * (uint32_t)lane
                                         : 0x80000000u;
          } else {
            const uint32_t row = (uint32_t)(16 * c + col), k = (uint32_t)j * KD + KG * (uint32_t)g;
            off = (jv && row < (uint32_t)rows_here && k < (uint32_t)p.K)
                      ? (row * (uint32_t)ldw + k) * (uint32_t)ES : 0x80000000u;
          }
          wq[u][c] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, kNT));
        }
        if constexpr (!XL) {
#pragma unroll
          for (int e = 0; e < NE; ++e)
#pragma unroll
            for (int b = 0; b < MB; ++b) {
              const uint32_t k = (uint32_t)j * KD + KG * (uint32_t)g + 8u * e;
              const uint32_t row = (uint32_t)(16 * b + col);
              const uint32_t off = (jv && row < (uint32_t)p.M && k < (uint32_t)p.K)
                                       ? (row * (uint32_t)p.ldx + k) * 2u : 0x80000000u;
              xq[u][e][b] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
            }
        }
      }
      // EAGER: the whole slice's loads stay ahead of its MFMAs
      if constexpr (EAGER) __builtin_amdgcn_sched_barrier(0);
      if constexpr (XL)
        if (c0 == 0) publish(std::integral_constant<int, CPW * CT>{});
#pragma unroll
      for (int u = 0; u < CPW; ++u)
#pragma unroll
        for (int e = 0; e < NE; ++e) {
          v4u xa[MB];
          if constexpr (XL) {
            // only the lanes of rows < M read (the others hold zeros)
            const int64_t k = (int64_t)(c0 + wave + KW * u) * KD + KG * g + 8 * e;
            xa[0] = v4u{0u, 0u, 0u, 0u};
            if (xrow && k < kp) xa[0] = *reinterpret_cast<const v4u*>(xs + col * xlp + k);
          } else {
#pragma unroll
            for (int b = 0; b < MB; ++b) xa[b] = xq[u][e][b];
          }
#pragma unroll
          for (int c = 0; c < CT; ++c) {
            v4u wb;
            if constexpr (WT == DT_I8)
              wb = __builtin_bit_cast(v4u, PK ? x8x8_to_v8h(wq[u][c][2 * e], wq[u][c][2 * e + 1])
                                           : i8x8_to_v8h(wq[u][c][2 * e], wq[u][c][2 * e + 1]));
            else
              wb = wq[u][c];
#pragma unroll
            for (int b = 0; b < MB; ++b) acc[b][c] = gv_mfma<WT>(xa[b], wb, acc[b][c]);
          }
        }
    }
  } else {
    // software pipelined over two register sets: slice i + 1's loads are in
    // flight while slice i is computed.  Loads past the last chunk read zero
    // (no memory traffic); computes past it are skipped.
    WFrag wa, wb;
    XFrag xa, xb;
    issue(0, wa, xa);
    issue(STEP, wb, xb);
    if constexpr (XL) publish(std::integral_constant<int, 2 * CPW * CT>{});
    for (int c0 = 0; c0 < kchunks; c0 += 2 * STEP) {
      compute(c0, wa, xa);
      issue(c0 + 2 * STEP, wa, xa);
      if (c0 + STEP < kchunks) compute(c0 + STEP, wb, xb);
      issue(c0 + 3 * STEP, wb, xb);
    }
  }

  // reduce the KW waves' partial tiles through LDS, one row block at a
  // time; thread t finalises (c, l, r) = (t / 256, (t / 4) % 64, t % 4).
  // The output has the activations' type (f16 for int8 and f16 weights,
  // bf16 for bf16).
  __shared__ float red[KW][CT][64][4];
  uint16_t* y = reinterpret_cast<uint16_t*>(p.y);
  if (few_rows) {
    // rows 0..3 of a 16-row block are lanes 0..15 of every tile: only those
    // go through LDS, and the first 64 CT threads finalise (c, l, r) =
    // (t / 64, (t / 4) % 16, t % 4), summing the waves in the same order as
    // the full reduction (identical results).
    float(*red4)[CT][16][4] = reinterpret_cast<float(*)[CT][16][4]>(&red[0][0][0][0]);
    if (lane < 16)
#pragma unroll
      for (int c = 0; c < CT; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) red4[wave][c][lane][r] = acc[0][c][r];
    __syncthreads();
    if (tid < 64 * CT) {
      const int c = tid >> 6, l = (tid >> 2) & 15, r = tid & 3;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) s += red4[w][c][l][r];
      const int64_t n = (int64_t)(t0 + c) * 16 + l;
      if (r < p.M && n < p.N) {
        const float v = has_scale ? s * sc[0] : s;
        const uint16_t h = WT == DT_BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
        y[(int64_t)r * p.ldy + n] = p.gate ? silu_mul_h(gv[0][0], h) : h;
      }
    }
    return;
  }
  // s * scale[n] in binary32 (an f16 scale widened exactly), rounded, gated
  auto finish = [&](int b, int i, int m, int64_t n, float s) {
    const float v = has_scale ? s * sc[i] : s;
    const uint16_t h = WT == DT_BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
    y[(int64_t)m * p.ldy + n] = p.gate ? silu_mul_h(gv[b][i], h) : h;
  };
#pragma unroll
  for (int b = 0; b < MB; ++b) {
    if (b > 0) __syncthreads();  // the previous block's sums are read
#pragma unroll
    for (int c = 0; c < CT; ++c)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[wave][c][lane][r] = acc[b][c][r];
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NSC; ++i) {
      const int e = tid + NT * i;
      if (e >= CT * 256) break;
      const int c = e >> 8, l = (e >> 2) & 63, r = e & 3;
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < KW; ++w) s += red[w][c][l][r];
      const int m = 16 * b + 4 * (l >> 4) + r;
      const int64_t n = (int64_t)(t0 + c) * 16 + (l & 15);
      if (m < p.M && n < p.N) {
        if (parts > 1)
          __hip_atomic_store(p.part + ((int64_t)part * p.M + m) * p.N + n, s, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        else
          finish(b, i, m, n, s);
      }
    }
  }
  if (parts == 1) return;
  // K split.  The partials, the counters and the reads of the partials are
  // device-scope atomic accesses, which the hardware keeps coherent across
  // the XCDs' L2s (written through, read past them); a device-scope fence
  // would instead write back and invalidate the whole L2 of the XCD, per
  // workgroup, which measured 10-30x slower.  Each wave waits for its
  // partial stores to complete before the barrier, so the part is counted
  // in only once every partial of the workgroup is visible; the workgroup
  // that counts last (its count returned before any of its partial loads
  // issue) finishes the outputs, adding the parts in part order whichever
  // finished last (the result does not depend on scheduling).  No
  // workgroup waits for another.
  //
  // What this relies on (gfx942 / gfx950, the AMDGPU memory model's code
  // sequences for agent scope): an agent-scope atomic store is a store
  // with the device-coherence bit set, written through the XCD's L2, and a
  // store's vmcnt decrement means it has been acknowledged at that
  // coherence point -- the model's own release sequence ("buffer_wbl2;
  // s_waitcnt vmcnt(0); store") rests on the same fact, its L2 write-back
  // being needed only for cached (non-atomic) earlier stores, of which
  // there are none here; an agent-scope atomic load bypasses the L2, so no
  // acquire invalidate is needed for loads that are all atomic.  GFX10+
  // counts stores separately (vscnt), where vmcnt(0) would not wait for
  // them: the guard below keeps this protocol to the gfx9 targets.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "split decode GEMV: the last-arriver protocol is written for gfx942 / gfx950 (vmcnt counts stores)"
#endif
  __shared__ int is_last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0)
    is_last = __hip_atomic_fetch_add(p.cnt + grp, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (unsigned)(parts - 1);
  __syncthreads();
  if (!is_last) return;
#pragma unroll
  for (int b = 0; b < MB; ++b)
#pragma unroll
    for (int i = 0; i < NSC; ++i) {
      const int e = tid + NT * i;
      if (e >= CT * 256) break;
      const int c = e >> 8, l = (e >> 2) & 63, r = e & 3;
      const int m = 16 * b + 4 * (l >> 4) + r;
      const int64_t n = (int64_t)(t0 + c) * 16 + (l & 15);
      if (m < p.M && n < p.N) {
        float* q = p.part + (int64_t)m * p.N + n;
        const int64_t stride = p.M * p.N;
        float s = __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int k = 1; k < parts; ++k)
          s += __hip_atomic_load(q + k * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        finish(b, i, m, n, s);
      }
    }
  if (tid == 0) __hip_atomic_store(p.cnt + grp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Build the fragment-packed image from a K-contiguous [N][K] int8 weight:
// packed block (t, j) byte 256*g + 16*c + i = W[n = 16t + c][k = 64j + 16g + i]
// ^ 0x80 (excess-128; 0x80, i.e. zero, beyond N or K).  One thread per
// 16-byte run (t, j, g, c).
__global__ void __launch_bounds__(256) gemv_pack_kernel(const int8_t* w, int64_t ldw, int64_t N,
                                                        int64_t K, int kchunks, int8_t* out) {
  const int64_t ntiles = (N + 15) / 16;
  const int64_t runs = ntiles * kchunks * 64;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < runs; q += (int64_t)gridDim.x * 256) {
    const int64_t blk = q >> 6;
    const int lane = (int)(q & 63);
    const int64_t t = blk / kchunks, j = blk - t * kchunks;
    const int c = lane & 15, g = lane >> 4;
    const int64_t n = t * 16 + c, k0 = j * 64 + 16 * g;
    uint8_t v[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
      v[i] = (uint8_t)(((n < N && k0 + i < K) ? (uint8_t)w[n * ldw + k0 + i] : 0u) ^ 0x80u);
    *reinterpret_cast<v4u*>(out + blk * 1024 + 16 * lane) = *reinterpret_cast<const v4u*>(v);
  }
}

int64_t gemv_packed_bytes(int64_t N, int64_t K) {
  return ((N + 15) / 16) * ((K + 63) / 64) * 1024;
}

// The 16-bit (f16 / bf16) fragment-packed image from a K-contiguous [N][K]
// weight: block (t, j) bytes 256*g + 16*c .. + 15 = W[n = 16t + c][k = 32j +
// 8g + (0..7)], zero beyond N or K.  One thread per 16-byte run.
__global__ void __launch_bounds__(256) gemv_pack16_kernel(const uint16_t* w, int64_t ldw, int64_t N,
                                                          int64_t K, int kchunks, uint16_t* out) {
  const int64_t ntiles = (N + 15) / 16;
  const int64_t runs = ntiles * kchunks * 64;
  for (int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x; q < runs; q += (int64_t)gridDim.x * 256) {
    const int64_t blk = q >> 6;
    const int lane = (int)(q & 63);
    const int64_t t = blk / kchunks, j = blk - t * kchunks;
    const int c = lane & 15, g = lane >> 4;
    const int64_t n = t * 16 + c, k0 = j * 32 + 8 * g;
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (n < N && k0 + i < K) ? w[n * ldw + k0 + i] : (uint16_t)0;
    *reinterpret_cast<v4u*>(out + blk * 512 + 8 * lane) = *reinterpret_cast<const v4u*>(v);
  }
}

int64_t gemv_packed16_bytes(int64_t N, int64_t K) {
  return ((N + 15) / 16) * ((K + 31) / 32) * 1024;
}

int launch_gemv_pack16(const uint16_t* w, int64_t ldw, int64_t N, int64_t K, uint16_t* out, hipStream_t s) {
  const int kchunks = (int)((K + 31) / 32);
  const int64_t runs = ((N + 15) / 16) * kchunks * 64;
  int64_t blocks = (runs + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  gemv_pack16_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(w, ldw, N, K, kchunks, out);
  return HXI_OK;
}

int launch_gemv_pack(const int8_t* w, int64_t ldw, int64_t N, int64_t K, int8_t* out, hipStream_t s) {
  const int kchunks = (int)((K + 63) / 64);
  const int64_t runs = ((N + 15) / 16) * kchunks * 64;
  int64_t blocks = (runs + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  gemv_pack_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(w, ldw, N, K, kchunks, out);
  return HXI_OK;
}

typedef void (*GemvStreamLaunch)(const GemvArgs&, const void*, int64_t, int, hipStream_t);
template <int CT, int KW, int CPW, int XS, bool PIPE, int WT, int MB = 1, bool PK = (WT == DT_I8),
          bool SPLIT = false, bool EAGER = false>
static void gemv_stream_one(const GemvArgs& a, const void* w, int64_t ldw, int kchunks, hipStream_t s) {
  constexpr int KD = WT == DT_I8 ? 64 : 32;
  const int64_t ntiles = (a.N + 15) / 16;
  const int64_t blocks = (ntiles + CT - 1) / CT * a.parts;
  const size_t lds = XS != XS_NONE ? (size_t)a.M * (((int64_t)kchunks * KD + 511) / 512 * 512 + 8) * 2 : 0;
  gemv_stream_kernel<CT, KW, CPW, XS, WT, PK, PIPE, MB, SPLIT, EAGER>
      <<<dim3((unsigned)blocks), dim3(64 * KW), lds, s>>>(a, w, ldw, kchunks);
}
struct GemvStreamEntry {
  GemvConfig cfg;
  GemvStreamLaunch fn[6];  // int8 (packed image), f16, bf16, int8 (in place), f16 / bf16 (packed image)
};
#define HX_GV(CT, KW, CPW, XS, PIPE)                                                                     \
  {&gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_I8>, &gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_F16>, \
   &gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_BF16>, &gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_I8, 1, false>, \
   &gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_F16, 1, true>, &gemv_stream_one<CT, KW, CPW, XS, PIPE, DT_BF16, 1, true>}
#define HX_GS(CT, KW, CPW)                                                                          \
  {&gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, 1, true, true>,                              \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, 1, false, true>,                            \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, 1, false, true>,                           \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, 1, false, true>,                             \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, 1, true, true>,                             \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, 1, true, true>}
#define HX_GE(CT, KW, CPW, SP)                                                                      \
  {&gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, 1, true, SP, true>,                          \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, 1, false, SP, true>,                        \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, 1, false, SP, true>,                       \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, 1, false, SP, true>,                         \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, 1, true, SP, true>,                         \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, 1, true, SP, true>}
#define HX_GSR(CT, KW, CPW, MB)                                                                     \
  {&gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB, true, true, true>,                       \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB, false, true, true>,                     \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB, false, true, true>,                    \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB, false, true, true>,                      \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB, true, true, true>,                      \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB, true, true, true>}
#define HX_GRE(CT, KW, CPW, MB)                                                                     \
  {&gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB, true, false, true>,                      \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB, false, false, true>,                    \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB, false, false, true>,                   \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB, false, false, true>,                     \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB, true, false, true>,                     \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB, true, false, true>}
#define HX_GR(CT, KW, CPW, MB)                                                                      \
  {&gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB>,                                        \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB>,                                       \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB>,                                      \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_I8, MB, false>,                                 \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_F16, MB, true>,                                 \
   &gemv_stream_one<CT, KW, CPW, XS_NONE, false, DT_BF16, MB, true>}
// xl configs (activations staged in LDS) take M <= 4 with the staged rows
// within 64 KiB of LDS; outside that they run as their register-staged base
// config (the `base` index).  The `_p` config is software pipelined over
// two K slices.  `rows` configs hold mb blocks of 16 activation rows; a
// config whose blocks cannot hold M runs as the row-block default.
static const GemvStreamEntry kGemvStream[] = {
    {{2, 8, "packed_ct2_kw8", 0, 0, 1}, HX_GV(2, 8, 8, XS_NONE, false)},
    {{1, 8, "packed_ct1_kw8", 0, 1, 1}, HX_GV(1, 8, 8, XS_NONE, false)},
    {{4, 8, "packed_ct4_kw8", 0, 2, 1}, HX_GV(4, 8, 4, XS_NONE, false)},
    {{2, 4, "packed_ct2_kw4", 0, 3, 1}, HX_GV(2, 4, 8, XS_NONE, false)},
    {{1, 4, "packed_ct1_kw4", 0, 4, 1}, HX_GV(1, 4, 16, XS_NONE, false)},
    {{1, 8, "packed_ct1_kw8_xl", 1, 1, 1}, HX_GV(1, 8, 8, XS_REG, false)},
    {{2, 8, "packed_ct2_kw8_xl", 1, 0, 1}, HX_GV(2, 8, 8, XS_REG, false)},
    {{1, 16, "packed_ct1_kw16_xl", 1, 1, 1}, HX_GV(1, 16, 4, XS_REG, false)},
    // 16 waves over K keep the 4-tile activation reuse of ct4 while putting
    // 4x more waves (and weight bytes in flight) on the CUs it occupies
    {{4, 16, "packed_ct4_kw16", 0, 8, 1}, HX_GV(4, 16, 2, XS_NONE, false)},
    // four tiles with every K chunk of K = 4096 int8 in flight at once (one
    // round trip to memory) over 16 or 8 waves
    {{4, 16, "packed_ct4_kw16_c4", 0, 9, 1}, HX_GV(4, 16, 4, XS_NONE, false)},
    {{4, 8, "packed_ct4_kw8_c8", 0, 10, 1}, HX_GV(4, 8, 8, XS_NONE, false)},
    {{1, 8, "packed_ct1_kw8_xd", 1, 1, 1}, HX_GV(1, 8, 8, XS_DMA, false)},
    // software pipelined: f16/bf16 weights with K spanning several slices
    // (27.5 against 31.1 us at M = 1, N = K = 8192 f16); no int8 shape gains
    {{1, 16, "packed_ct1_kw16_xl_p", 1, 1, 1}, HX_GV(1, 16, 4, XS_REG, true)},
    {{1, 8, "rows2_ct1_kw8", 0, 13, 2}, HX_GR(1, 8, 8, 2)},
    {{2, 8, "rows2_ct2_kw8", 0, 14, 2}, HX_GR(2, 8, 4, 2)},
    {{1, 8, "rows4_ct1_kw8", 0, 15, 4}, HX_GR(1, 8, 4, 4)},
    {{2, 8, "rows4_ct2_kw8", 0, 16, 4}, HX_GR(2, 8, 4, 4)},
    {{4, 8, "rows4_ct4_kw8", 0, 17, 4}, HX_GR(4, 8, 2, 4)},
    {{1, 4, "rows4_ct1_kw4", 0, 18, 4}, HX_GR(1, 4, 8, 4)},
    // three tiles: 230 workgroups at N = 11008 (four tiles leave 172 of 256
    // CUs busy, two re-read the activation fragments twice as often)
    {{3, 8, "packed_ct3_kw8", 0, 19, 1}, HX_GV(3, 8, 8, XS_NONE, false)},
    {{3, 16, "packed_ct3_kw16", 0, 20, 1}, HX_GV(3, 16, 4, XS_NONE, false)},
    // three tiles with two or four row blocks: one workgroup per CU at
    // N = 11008 for 16 < M <= 32 (two blocks) or 64 (four)
    {{3, 8, "rows2_ct3_kw8", 0, 21, 2}, HX_GR(3, 8, 4, 2)},
    {{3, 8, "rows4_ct3_kw8", 0, 22, 4}, HX_GR(3, 8, 2, 4)},
    // sixteen waves over K: more weight bytes in flight per CU when N gives
    // one tile per CU (the FFN's down projection, N = 4096, K = 11008)
    {{1, 16, "rows2_ct1_kw16", 0, 23, 2}, HX_GR(1, 16, 4, 2)},
    {{1, 16, "packed_ct1_kw16", 0, 24, 1}, HX_GV(1, 16, 4, XS_NONE, false)},
    // K split over two or four workgroups per tile group (M > 4): each
    // workgroup reads 1/parts of the activation rows for `ct` tiles, so the
    // activation fragments it loads per weight byte drop by the tile count
    // while the workgroup count stays at one per CU (N = 4096: 128 x 2 and
    // 64 x 4; N = 11008: 115 x 2)
    {{2, 16, "packed_ct2_kw16_s2", 0, 0, 1, 2}, HX_GS(2, 16, 4)},
    {{4, 16, "packed_ct4_kw16_s4", 0, 8, 1, 4}, HX_GS(4, 16, 2)},
    {{6, 16, "packed_ct6_kw16_s2", 0, 20, 1, 2}, HX_GS(6, 16, 2)},
    // at most 128 tiles (N <= 2048): one or two tiles per workgroup with K
    // split in two or four, 2x the workgroups of one tile each
    {{1, 16, "packed_ct1_kw16_s2", 0, 24, 1, 2}, HX_GS(1, 16, 4)},
    {{2, 16, "packed_ct2_kw16_s4", 0, 0, 1, 4}, HX_GS(2, 16, 4)},
    // every slice load issued before the slice's first MFMA (the compiler
    // otherwise spreads the loads among the MFMAs, about 6 of a wave's 20
    // in flight for ct3_kw16): 1-3% faster on these shapes (interleaved A/B,
    // int8 packed image; N = 11008, K = 4096, M = 1 / 4 / 8 / 12 / 16: 9.48 /
    // 9.45 / 9.55 / 9.86 / 10.39 against 9.55 / 9.67 / 9.98 / 10.46 / 11.06 us
    // for ct3_kw16; N = 4096, K = 11008, M = 8 / 12 / 16: ct1_kw16 11.84 /
    // 13.56 / 15.03 against 12.35 / 13.99 / 16.07, ct4_kw16_s4 12.78 / 13.09 /
    // 13.38 against 12.95 / 13.27 / 13.62); it lost on ct4_kw16, ct3_kw8 at
    // 16 rows and ct2_kw16_s2
    {{3, 16, "packed_ct3_kw16_e", 0, 30, 1}, HX_GE(3, 16, 4, false)},
    {{1, 8, "packed_ct1_kw8_e", 0, 31, 1}, HX_GE(1, 8, 8, false)},
    {{1, 16, "packed_ct1_kw16_e", 0, 32, 1}, HX_GE(1, 16, 4, false)},
    {{4, 16, "packed_ct4_kw16_s4_e", 0, 8, 1, 4}, HX_GE(4, 16, 2, true)},
    // two row blocks (16 < M <= 32) with K split over workgroups and the
    // loads issued ahead
    {{4, 16, "rows2_ct4_kw16_s4_e", 0, 8, 2, 4}, HX_GSR(4, 16, 2, 2)},
    {{2, 16, "rows2_ct2_kw16_s2_e", 0, 0, 2, 2}, HX_GSR(2, 16, 2, 2)},
    // four row blocks (32 < M <= 64), loads issued ahead: three tiles over
    // sixteen waves, and four tiles with K split in four (interleaved A/B
    // against the tiled W8A16 GEMM, int8 packed images rotating over 600 MB;
    // N = 11008, K = 4096, M = 33 / 48 / 64: 16.90 / 20.88 / 23.33 against
    // 21.03 / 22.35 / 22.62 us; N = 4096, K = 11008: 22.37 / 24.21 / 28.30
    // against 31.11 / 31.30 / 31.32, where the unsplit rows4_ct1_kw8 took
    // 37.5 / 44.4 / 50.0)
    {{3, 16, "rows4_ct3_kw16_e", 0, 22, 4}, HX_GRE(3, 16, 1, 4)},
    {{4, 8, "rows4_ct4_kw8_s4_e", 0, 17, 4, 4}, HX_GSR(4, 8, 2, 4)},
};
#undef HX_GR
#undef HX_GRE
#undef HX_GE
#undef HX_GSR
#undef HX_GS
#undef HX_GV
int gemv_packed_config_count() { return (int)(sizeof(kGemvStream) / sizeof(kGemvStream[0])); }
const GemvConfig* gemv_packed_config(int idx) {
  if (idx < 0 || idx >= gemv_packed_config_count()) return nullptr;
  return &kGemvStream[idx].cfg;
}

// Shared by the packed-image and in-place launches.
static int launch_gemv_stream(int cfg_idx, int wt, bool packed, const GemvArgs& a, const void* w,
                              int64_t ldw, hipStream_t s) {
  if (cfg_idx < 0 || cfg_idx >= gemv_packed_config_count()) return HXI_ERR_ARG;
  if (a.M < 1 || a.M > kGemvMaxRows) return HXI_ERR_SHAPE;
  // a config whose row blocks cannot hold M runs as the row-block default
  if (a.M > 16 * kGemvStream[cfg_idx].cfg.mb) cfg_idx = gemv_rows_default(a.M, a.N, a.K);
  const int slot = wt == DT_I8 ? (packed ? 0 : 3) : wt == DT_F16 ? (packed ? 4 : 1) : wt == DT_BF16 ? (packed ? 5 : 2) : -1;
  if (slot < 0) return HXI_ERR_ARG;
  const int64_t kd = wt == DT_I8 ? 64 : 32;
  const int64_t kchunks = (a.K + kd - 1) / kd;
  const int64_t ct = kGemvStream[cfg_idx].cfg.ct;
  // 32-bit buffer offsets: one workgroup's weight range and the activation rows
  const int64_t wg_bytes = packed ? ct * kchunks * 1024 : 16 * ct * ldw * (wt == DT_I8 ? 1 : 2);
  if (wg_bytes >= ((int64_t)1 << 31) || a.M * a.ldx * 2 >= ((int64_t)1 << 31)) return HXI_ERR_SHAPE;
  if (kGemvStream[cfg_idx].cfg.xl && !gemv_xl_fits(kGemvStream[cfg_idx].cfg, a.M, a.K, wt))
    cfg_idx = kGemvStream[cfg_idx].cfg.base;
  const GemvConfig& c = kGemvStream[cfg_idx].cfg;
  GemvArgs v = a;
  v.parts = 1;
  if (c.split > 1) {
    if (!gemv_split_takes(c, a.M, a.N)) {
      cfg_idx = c.base;
    } else {
      v.parts = c.split;
      if (!v.part || !v.cnt) {
        const int rc = gemv_split_buffers(s, gemv_split_bytes(cfg_idx, a.M, a.N), &v.part, &v.cnt);
        if (rc) return rc;
      }
    }
  }
  kGemvStream[cfg_idx].fn[slot](v, w, ldw, (int)kchunks, s);
  return HXI_OK;
}
bool gemv_split_takes(const GemvConfig& c, int64_t M, int64_t N) {
  // M <= 4 takes the few-row reduction, which finishes in place
  return c.split > 1 && !c.xl && M > 4 && M <= 16 * c.mb &&
         ((N + 15) / 16 + c.ct - 1) / c.ct <= kGemvSplitCounters;
}
size_t gemv_split_bytes(int cfg, int64_t M, int64_t N) {
  const GemvConfig* c = gemv_packed_config(cfg);
  if (!c || !gemv_split_takes(*c, M, N)) return 0;
  return (size_t)c->split * (size_t)M * (size_t)N * 4;
}
bool gemv_xl_fits(const GemvConfig& c, int64_t M, int64_t K, int wt) {
  if (!c.xl) return true;
  const int64_t kd = wt == DT_I8 ? 64 : 32;
  return M <= 4 && M * (((K + kd - 1) / kd * kd + 511) / 512 * 512 + 8) * 2 <= 65536;
}
// Measured at M = 17..64 (tuner medians, rotating packed images): up to 32
// rows two row blocks over three tiles where that gives one workgroup per
// CU (int8 N = 11008, M = 17 / 24 / 32: 15.2 / 15.8 / 16.7 us against 17.1 /
// 19.9 / 23.4 for two tiles), two tiles above 256 tiles, the K split below
// on the down projection's shapes, else one tile over 16 waves (int8 N =
// 4096, K = 11008, before the split: 18.7 / 22.2 / 26.5 against 25.1 / 26.5
// / 29.6 over 8 waves); beyond 32 rows four row blocks (below).
int gemv_rows_default(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = (N + 15) / 16;
  // more than 128 and at most 256 tiles with K >= 8192 (the FFN's down
  // projection): two row blocks with K split over workgroups, loads issued
  // ahead -- two tiles over two parts up to 20 rows, four over four beyond
  // (4096 x 11008, M = 17 / 20 / 24 / 28 / 32: 14.81 / 15.74 / 16.82 /
  // 18.02 / 19.18 and 15.89 / 16.22 / 16.64 / 17.27 / 17.75 us against
  // 18.53 / 20.31 / 22.25 / 24.10 / 26.02 for one tile over 16 waves)
  if (M <= 32 && tiles > 128 && tiles <= 256 && K >= 8192) return M <= 20 ? 35 : 34;
  if (M <= 32) return (tiles + 255) / 256 == 3 ? 21 : tiles > 256 ? 14 : 23;
  // Beyond 32 rows, four row blocks with the loads issued ahead: four tiles
  // with K split in four on the down projection's shapes, three tiles over
  // sixteen waves where that gives one workgroup per CU (N = 11008).  The
  // products route only these shapes here (gemv_rows_route); elsewhere the
  // four-block kernels lost to the tiled GEMM.
  if (tiles > 128 && tiles <= 256 && K >= 8192) return 37;
  if ((tiles + 255) / 256 == 3) return 36;
  return N >= 160 * 64 ? 17 : 15;
}
int launch_gemv_packed(int cfg_idx, const GemvArgs& a, const int8_t* packed, hipStream_t s) {
  return launch_gemv_stream(cfg_idx, DT_I8, true, a, packed, 0, s);
}
int launch_gemv_packed16(int cfg_idx, int wt, const GemvArgs& a, const void* packed, hipStream_t s) {
  if (wt != DT_F16 && wt != DT_BF16) return HXI_ERR_ARG;
  return launch_gemv_stream(cfg_idx, wt, true, a, packed, 0, s);
}
const char* gemv_hw_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const int64_t es = wt == DT_I8 ? 1 : 2;
  if (a.M < 1 || a.M > kGemvMaxRows || a.N < 1 || a.K < 1) return "row-count";
  if (a.K % 8 != 0) return "k-granularity";
  if ((ldw * es) % 16 != 0 || (a.ldx * 2) % 16 != 0) return "row-stride";
  if (!al16(a.x) || !al16(w)) return "unaligned-base";
  if ((int64_t)64 * ldw * es >= ((int64_t)1 << 31) || a.M * a.ldx * 2 >= ((int64_t)1 << 31))
    return "offset-range";
  return nullptr;
}
int launch_gemv_hw(int cfg_idx, int wt, const GemvArgs& a, const void* w, int64_t ldw, hipStream_t s) {
  if (wt != DT_F16 && wt != DT_BF16 && wt != DT_I8) return HXI_ERR_ARG;
  if (gemv_hw_refusal(wt, a, w, ldw)) return HXI_ERR_SHAPE;
  return launch_gemv_stream(cfg_idx, wt, false, a, w, ldw, s);
}

// ---------------------------------------------------------------------------
// One activation row against the rows of a K-contiguous matrix:
//   y[n] = RNE( (sum_k W[n][k] * x[k]) * s[n] ),  binary32 accumulation,
// for the decode of one row against an [N][K] weight read in place and for
// hx_matmul with N = 1 (A's rows against b).  The MFMA GEMV's fragment
// layout reads such a weight as sixteen 64-byte runs per wave load; here
// each wave owns whole rows and reads them in contiguous KiBs (lane l holds
// bytes 16l .. 16l + 15 of each), which streams like the packed image.  x is
// staged once per workgroup in LDS (zero past K); products accumulate with
// v_dot2 (two f16 / bf16 products and the running sum per instruction; int8
// widened to f16 exactly first), then a butterfly adds the 64 lanes.
// Wave w of workgroup b takes rows n = 4b + w + 4 G t (G workgroups); all of
// a row's loads are in flight together, and the next row's are issued
// before this row's products.
// acc + sum of the eight products of two 16-byte vectors of f16 (bf16)
// pairs, in element order.  The components are copied into scalars first:
// hipcc compiled __builtin_bit_cast of a component expression (w.y) as a
// cast of component 0.
template <int WT>
__device__ __forceinline__ float dot8(v4u w, v4u x, float acc) {
  const uint32_t w0 = w[0], w1 = w[1], w2 = w[2], w3 = w[3];
  const uint32_t x0 = x[0], x1 = x[1], x2 = x[2], x3 = x[3];
  if constexpr (WT == DT_BF16) {
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, w0), __builtin_bit_cast(v2bf, x0), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, w1), __builtin_bit_cast(v2bf, x1), acc, false);
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, w2), __builtin_bit_cast(v2bf, x2), acc, false);
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2bf, w3), __builtin_bit_cast(v2bf, x3), acc, false);
  } else {
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, w0), __builtin_bit_cast(v2h, x0), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, w1), __builtin_bit_cast(v2h, x1), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, w2), __builtin_bit_cast(v2h, x2), acc, false);
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2h, w3), __builtin_bit_cast(v2h, x3), acc, false);
  }
}

template <int WT>
__global__ void __launch_bounds__(256) rowdot_kernel(GemvArgs p, const void* wsrc, int64_t ldw) {
  constexpr int ES = WT == DT_I8 ? 1 : 2;   // weight element bytes
  constexpr int EPL = 16 / ES;              // weight elements per lane load
  constexpr int CK = 64 * EPL;              // k per wave load (chunk)
  constexpr int U = WT == DT_I8 ? 8 : 16;   // chunks per row held at once
  extern __shared__ __attribute__((aligned(16))) uint16_t xs[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kc = (int)((p.K + CK - 1) / CK);  // chunks per row (<= U)
  // stage x (K halves, 16-byte groups; K % 8 == 0), zero up to U * CK: the
  // chunk loop always runs U chunks (fully unrolled; chunks past the row
  // load zeros through the buffer range and add exact zeros)
  {
    const uint16_t* x = reinterpret_cast<const uint16_t*>(p.x);
    for (int64_t i = tid; i < (int64_t)U * CK / 8; i += 256) {
      v4u v = v4u{0u, 0u, 0u, 0u};
      if (8 * i < p.K) v = *reinterpret_cast<const v4u*>(x + 8 * i);
      *reinterpret_cast<v4u*>(xs + 8 * i) = v;
    }
  }
  __syncthreads();
  const int64_t rstep = (int64_t)gridDim.x * 4;
  const char* wb = reinterpret_cast<const char*>(wsrc);
  auto issue = [&](int64_t n, v4u (&q)[U]) {
    const bool nin = n < p.N;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(wb + (nin ? n : 0) * ldw * ES), 0, nin ? (int)(p.K * ES) : 0, 0x00020000);
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const uint32_t off = (uint32_t)(c * CK + EPL * lane) * ES;
      q[c] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, c < kc ? (int)off : (int)0x80000000, 0, 2));
    }
  };
  v4u qa[U], qb[U];
  int64_t n = (int64_t)blockIdx.x * 4 + wave;
  issue(n, qa);
  for (; n < p.N; n += rstep) {
    issue(n + rstep, qb);
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < U; ++c) {
      const uint16_t* xl = xs + c * CK + EPL * lane;
      if constexpr (WT == DT_I8) {
        const v4u x0 = *reinterpret_cast<const v4u*>(xl), x1 = *reinterpret_cast<const v4u*>(xl + 8);
        const v4u q = qa[c];
        const uint32_t q0 = q[0], q1 = q[1], q2 = q[2], q3 = q[3];
        acc = dot8<DT_F16>(__builtin_bit_cast(v4u, i8x8_to_v8h(q0, q1)), x0, acc);
        acc = dot8<DT_F16>(__builtin_bit_cast(v4u, i8x8_to_v8h(q2, q3)), x1, acc);
      } else {
        acc = dot8<WT>(qa[c], *reinterpret_cast<const v4u*>(xl), acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0) {
      const float v = gv_scaled(p, n, acc);
      reinterpret_cast<uint16_t*>(p.y)[n] = WT == DT_BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
    }
#pragma unroll
    for (int c = 0; c < U; ++c) qa[c] = qb[c];
  }
}

const char* rowdot_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw) {
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15u) == 0; };
  const int64_t es = wt == DT_I8 ? 1 : 2;
  const int64_t ck = 64 * (16 / es);
  if (a.M != 1 || a.N < 1 || a.K < 1) return "row-count";
  if (a.K % (16 / es) != 0) return "k-granularity";
  if ((a.K + ck - 1) / ck > (wt == DT_I8 ? 8 : 16)) return "k-extent";  // K <= 8192
  if ((ldw * es) % 16 != 0) return "row-stride";
  if (!al16(a.x) || !al16(w)) return "unaligned-base";
  return nullptr;
}

int launch_rowdot(int wt, const GemvArgs& a, const void* w, int64_t ldw, hipStream_t s) {
  if (rowdot_refusal(wt, a, w, ldw)) return HXI_ERR_SHAPE;
  const size_t lds = 8192 * 2;  // U chunks of x: 8192 halves
  // about two workgroups per CU, each wave then taking N / 2048 rows
  const int64_t blocks = std::min<int64_t>((a.N + 3) / 4, 512);
  switch (wt) {
    case DT_F16: rowdot_kernel<DT_F16><<<dim3((unsigned)blocks), dim3(256), lds, s>>>(a, w, ldw); break;
    case DT_BF16: rowdot_kernel<DT_BF16><<<dim3((unsigned)blocks), dim3(256), lds, s>>>(a, w, ldw); break;
    case DT_I8: rowdot_kernel<DT_I8><<<dim3((unsigned)blocks), dim3(256), lds, s>>>(a, w, ldw); break;
    default: return HXI_ERR_ARG;
  }
  return HXI_OK;
}

// ---------------------------------------------------------------------------
// Weights in the linalg [K][N] orientation (N contiguous), read in place: no
// transpose of the weight.  f16 / bf16 weights, or int8 (W8A16, f16
// activations).
//
// A lane load is 16 bytes of one row: NQ = 8 (f16/bf16) or 16 (int8)
// consecutive columns.  Workgroup (column block b, K part s) covers the
// CB = 16 NQ columns CB*b .. CB*b + CB - 1.  Lane l = 16g + c of a wave
// loads, for K chunk j (32 k), the eight rows W[32j + 8g + r][CB*b + NQ*c +
// (0..NQ-1)], r = 0..7 (a wave load is four runs of 16 x 16 bytes), and
// transposes that block in registers: for each q < NQ it then holds column
// CB*b + NQ*c + q at k = 32j + 8g + (0..7), which is the
// v_mfma_f32_16x16x32 B operand of lane l for the "tile" of the 16 columns
// {CB*b + NQ*c' + q : c' = 0..15}.  f16/bf16: 32 v_perm_b32 per chunk move
// halves; int8: one v_perm_b32 per pair of rows puts the two bytes of a
// column into the low bytes of two halves, the XOR with 0x64806480 makes
// them 1024 + (b ^ 128) exactly, and subtracting 1152 leaves the signed
// value.  The activation operand is the row-fragment x[c][32j + 8g +
// (0..7)] (rows >= M read zero), shared by the NQ tiles.  Accumulator
// register i of tile q in lane l is Y[4g + i][CB*b + NQ*c + q].
// The KW waves of a workgroup and the S K parts split the chunks (wave w of
// part s takes chunks j = s*KW + w + S*KW*t); the waves reduce through LDS,
// and with S > 1 each part writes binary32 partials [S][M][N] that
// gemv_kn_combine_kernel sums, scales and rounds.
template <int WT, int KW, int U>
__global__ void __launch_bounds__(64 * KW) gemv_kn_kernel(GemvArgs p, const void* wsrc, int64_t ldw, int kchunks,
                                                          float* part) {
  constexpr int ES = WT == DT_I8 ? 1 : 2;  // weight element bytes
  constexpr int NQ = 16 / ES;              // columns per lane load
  constexpr int CB = 16 * NQ;              // columns per workgroup
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, g = lane >> 4;
  const int64_t n0 = (int64_t)blockIdx.x * CB;
  const int S = gridDim.y, sp = blockIdx.y;
  const int P = S * KW;  // chunk stride
  // the weight rows of this column block: byte offset (k * ldw + NQ c + q) * ES
  const char* wb = reinterpret_cast<const char*>(wsrc) + n0 * ES;
  const int64_t wbytes = ((p.K - 1) * ldw + (p.N - n0)) * ES;  // to the last element of the block's range
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wb, 0, (int)min(wbytes, (int64_t)0x7fffffff), 0x00020000);
  const __amdgpu_buffer_rsrc_t rx =
      __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, (int)(p.M * p.ldx * 2), 0x00020000);
  const bool xrow = c < p.M;
  const bool cin = n0 + NQ * c < p.N;  // this lane's column run starts inside N
  constexpr int kNT = 2;

  v4f acc[NQ];
#pragma unroll
  for (int q = 0; q < NQ; ++q) acc[q] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int j0 = sp * KW + wave; j0 < kchunks; j0 += P * U) {
    v4u wr[U][8];
    v4u xa[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = j0 + P * u;
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint32_t k = (uint32_t)j * 32u + 8u * g + r;
        const uint32_t off = (j < kchunks && cin && k < (uint32_t)p.K)
                                 ? (k * (uint32_t)ldw + (uint32_t)NQ * c) * (uint32_t)ES : 0x80000000u;
        wr[u][r] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rw, (int)off, 0, kNT));
      }
      const uint32_t kx = (uint32_t)j * 32u + 8u * g;
      const uint32_t offx = (j < kchunks && xrow && kx < (uint32_t)p.K)
                                ? ((uint32_t)c * (uint32_t)p.ldx + kx) * 2u : 0x80000000u;
      xa[u] = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)offx, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (WT == DT_I8) {
        typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
        const hf2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          // byte q & 3 of dword q >> 2 of rows 2pr (low half) and 2pr + 1 (high half)
          constexpr uint32_t Z = 0x0cu;  // selector of a zero byte
          const uint32_t bq = (uint32_t)(q & 3);
          const uint32_t sel = (Z << 24) | ((4u + bq) << 16) | (Z << 8) | bq;
          v4u t;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            const uint32_t d = __builtin_amdgcn_perm(wr[u][2 * pr + 1][q >> 2], wr[u][2 * pr][q >> 2], sel) ^ 0x64806480u;
            t[pr] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(hf2, d) - bias);
          }
          acc[q] = gv_mfma<DT_F16>(xa[u], t, acc[q]);
        }
      } else {
        // 8 x 8 transpose of halves: dword d of rows 2p, 2p+1 -> columns 2d, 2d+1
        v4u t[8];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr)
#pragma unroll
          for (int d = 0; d < 4; ++d) {
            const uint32_t a = wr[u][2 * pr][d], b = wr[u][2 * pr + 1][d];
            t[2 * d][pr] = __builtin_amdgcn_perm(b, a, 0x05040100u);      // low halves
            t[2 * d + 1][pr] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // high halves
          }
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = gv_mfma<WT>(xa[u], t[q], acc[q]);
      }
    }
  }

  // reduce the KW waves through LDS; thread t finalises (q, l, i) =
  // (e / 256, (e / 4) % 64, e % 4) for e = t, t + 64 KW, ...
  __shared__ float red[KW][NQ][64][4];
#pragma unroll
  for (int q = 0; q < NQ; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][q][lane][i] = acc[q][i];
  __syncthreads();
  for (int e = tid; e < NQ * 256; e += 64 * KW) {
    const int q = e >> 8, l = (e >> 2) & 63, i = e & 3;
    float sum = 0.f;
#pragma unroll
    for (int w = 0; w < KW; ++w) sum += red[w][q][l][i];
    const int m = 4 * (l >> 4) + i;
    const int64_t n = n0 + NQ * (l & 15) + q;
    if (m < p.M && n < p.N) {
      if (S > 1) {
        // plain stores: written through to memory they took 19.2 / 31.6 us
        // against 18.2 / 22.4 at M = 1 / 16 (int8, N = 11008)
        part[((int64_t)sp * p.M + m) * p.N + n] = sum;
      } else {
        const float v = gv_scaled(p, n, sum);
        reinterpret_cast<uint16_t*>(p.y)[(int64_t)m * p.ldy + n] = WT == DT_BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
      }
    }
  }
}

// Y[m][n] = RNE( (sum_s part[s][m][n]) * scale[n] ), parts summed in order.
template <int WT>
__global__ void __launch_bounds__(256) gemv_kn_combine_kernel(GemvArgs p, const float* part, int S) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= p.M * p.N) return;
  const int64_t m = t / p.N, n = t - m * p.N;
  float sum = 0.f;
  for (int s = 0; s < S; ++s) sum += part[(int64_t)s * p.M * p.N + t];
  const float v = gv_scaled(p, n, sum);
  reinterpret_cast<uint16_t*>(p.y)[m * p.ldy + n] = WT == DT_BF16 ? f32_to_bf16(v) : f32_to_f16_bits(v);
}

namespace {
constexpr int kKnWaves = 4, kKnUnroll = 2;
int kn_elem_bytes(int wt) { return wt == DT_I8 ? 1 : 2; }
}
const char* gemv_kn_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  const int es = kn_elem_bytes(wt);
  if (a.M < 1 || a.M > 16 || a.N < 1 || a.K < 1) return "row-count";
  if ((ldw * es) % 16 != 0 || (a.ldx * 2) % 16 != 0 || a.K % 8 != 0) return "row-stride";
  // whole 16-byte column runs: a load never straddles the end of a row
  if (a.N % (16 / es) != 0) return "n-granularity";
  if (!al16(a.x) || !al16(w)) return "unaligned-base";
  if (a.K * ldw * es >= ((int64_t)1 << 31) || a.M * a.ldx * 2 >= ((int64_t)1 << 31)) return "offset-range";
  return nullptr;
}
int gemv_kn_parts(int wt, const GemvArgs& a) {
  // about 256 workgroups (measured against 128 and 512: int8 11008x4096
  // 19.9 / 20.0 / 21.6 us, f16 4096^2 12.8 / 13.5 / 14.9 us at M = 1), each
  // wave with at least kKnUnroll chunks per part
  const int64_t cb = 16 * (16 / kn_elem_bytes(wt));
  const int64_t blocks = (a.N + cb - 1) / cb;
  const int64_t kchunks = (a.K + 31) / 32;
  int64_t S = (256 + blocks - 1) / blocks;
  S = std::min<int64_t>(S, kchunks / (kKnWaves * kKnUnroll));
  S = std::min<int64_t>(S, 64);
  S = std::min<int64_t>(S, ((((int64_t)1 << 31) - 1) / 4) / (a.M * a.N));  // partials' 32-bit offsets
  return (int)std::max<int64_t>(S, 1);
}
size_t gemv_kn_part_bytes(const GemvArgs& a, int parts) {
  return parts > 1 ? (size_t)parts * (size_t)(a.M * a.N) * sizeof(float) : 0;
}
template <int WT>
static void gemv_kn_launch(const GemvArgs& a, const void* w, int64_t ldw, int parts, float* part, hipStream_t s) {
  constexpr int CB = 16 * (16 / (WT == DT_I8 ? 1 : 2));
  const int kchunks = (int)((a.K + 31) / 32);
  const dim3 grid((unsigned)((a.N + CB - 1) / CB), (unsigned)parts);
  gemv_kn_kernel<WT, kKnWaves, kKnUnroll><<<grid, dim3(64 * kKnWaves), 0, s>>>(a, w, ldw, kchunks, part);
  if (parts > 1)
    gemv_kn_combine_kernel<WT><<<dim3((unsigned)((a.M * a.N + 255) / 256)), dim3(256), 0, s>>>(a, part, parts);
}
int launch_gemv_kn(int wt, const GemvArgs& a, const void* w, int64_t ldw, int parts, float* part, hipStream_t s) {
  if (wt != DT_F16 && wt != DT_BF16 && wt != DT_I8) return HXI_ERR_ARG;
  if (gemv_kn_refusal(wt, a, w, ldw) || parts < 1 || parts > 64 || (parts > 1 && !part)) return HXI_ERR_SHAPE;
  if (wt == DT_F16) gemv_kn_launch<DT_F16>(a, w, ldw, parts, part, s);
  else if (wt == DT_BF16) gemv_kn_launch<DT_BF16>(a, w, ldw, parts, part, s);
  else gemv_kn_launch<DT_I8>(a, w, ldw, parts, part, s);
  return HXI_OK;
}

typedef void (*GemvLaunch)(const GemvArgs&, hipStream_t);

template <int CT>
static void gemv_launch_one(const GemvArgs& a, hipStream_t s) {
  const int64_t tiles = (a.N + 16 * CT - 1) / (16 * CT);
  gemv_w8a16_kernel<CT><<<dim3((unsigned)tiles), dim3(256), 0, s>>>(a);
}

// Kernels for a K-contiguous [N][K] weight that is not registered (no packed
// image): 16*CT columns per workgroup, the four waves split K.
static const GemvLaunch kGemvNK[] = {&gemv_launch_one<1>, &gemv_launch_one<2>, &gemv_launch_one<4>};

const char* gemv_fast_refusal(const GemvArgs& a) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.M < 1 || a.M > 16 || a.N < 1 || a.K < 1) return "row-count";
  if (a.K % 16 != 0) return "k-granularity";
  if (a.ldw % 16 != 0 || (a.ldx * 2) % 16 != 0) return "row-stride";
  if (!al16(a.x) || !al16(a.w)) return "unaligned-base";
  if ((int64_t)64 * a.ldw >= ((int64_t)1 << 31)) return "offset-range";
  if ((int64_t)a.M * a.ldx * 2 >= ((int64_t)1 << 31)) return "offset-range";
  return nullptr;
}
bool gemv_fast_ok(const GemvArgs& a) { return gemv_fast_refusal(a) == nullptr; }
int gemv_raw_config(const GemvArgs& a) { return a.N >= 4096 ? 1 : 0; }
int launch_gemv_w8a16(const GemvArgs& a, hipStream_t s) {
  kGemvNK[gemv_raw_config(a)](a, s);
  return HXI_OK;
}

}  // namespace hx
