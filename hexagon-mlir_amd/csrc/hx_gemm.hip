// hx_gemm.hip -- MFMA GEMM family for gfx950: int8 x int8 -> int32,
// f16/bf16 x f16/bf16 -> f32, and f16 x int8 (W8A16, weights widened to f16
// in registers) -> f32, with fused epilogues (int32 store, per-row/per-column
// dequant to fp16, per-channel scale + residual, SwiGLU gate*up).
//
// What it replaces in hexagon-mlir (QHB = qcom_hexagon_backend):
//   * the HMX tile loop -- hmx-partition's (m,n) loop with K batches of up to
//     32 croutons per hmx_mma_f16 and a staged activation ring
//     (QHB/lib/Dialect/Hmx/Transforms/HmxPartitionPass.cpp:783-866, 2001-2066)
//     and the leaf itself (QHB/bin/runtime/hmx/src/HMXAPI.c:47-55);
//   * the HVX (i,k,j) generic that int8 and skinny matmuls fall back to
//     (QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:169-196);
//   * the fused read-out (HMXAPI.c:30-44, HMXLayout.c:692-999).
//
// Design (MI355X-first, not a translation of the crouton scheme):
//   * one workgroup per BMxBN output tile; a tile is split over WMxWN waves,
//     each owning (BM/WM)x(BN/WN) = TMxTN MFMA 32x32 sub-tiles whose
//     accumulators live in AGPRs for the whole K loop;
//   * K is walked in stages of 128 bytes of A per row; each stage of A and B
//     is loaded with 16-byte buffer loads (out-of-range rows and the K tail
//     read as zero from the buffer descriptor's range) into registers one
//     stage ahead and written to a double-buffered LDS ring, one barrier per
//     stage;
//   * LDS rows are 128 (or 64) bytes with the 16-byte chunk index XOR-swizzled
//     by the row so that the MFMA operand reads (16 bytes per lane, 32 rows)
//     and the stage writes are bank-conflict free;
//   * B is consumed K-contiguous ([N][K]), i.e. the weight image the resident
//     registry keeps -- the counterpart of the reference's pre-packed WH
//     crouton image (QHB/backend/hmx_weight_prepack.py:171-212);
//   * workgroup ids are renumbered so that each XCD (workgroups are dealt to
//     the 8 XCDs round robin) walks a compact block of tiles: the B strips of
//     that block stay resident in the XCD's L2 while its M-tiles go by.
#include "hx_device.hpp"
#include "hx_internal.hpp"
#include <type_traits>

namespace hx {

template <int MODE> struct ModeTraits;
template <> struct ModeTraits<GM_I8> {
  static constexpr int EA = 1, EB = 1, BK = 128, BROW = 128;
  typedef v16i Acc;
};
template <> struct ModeTraits<GM_F16> {
  static constexpr int EA = 2, EB = 2, BK = 64, BROW = 128;
  typedef v16f Acc;
};
template <> struct ModeTraits<GM_BF16> {
  static constexpr int EA = 2, EB = 2, BK = 64, BROW = 128;
  typedef v16f Acc;
};
template <> struct ModeTraits<GM_W8> {
  static constexpr int EA = 2, EB = 1, BK = 64, BROW = 64;
  typedef v16f Acc;
};

// Chunk swizzles.  For 128-byte rows, (row ^ row>>3) & 7 makes any 8 and any
// 16 consecutive rows reading the same logical chunk hit distinct bank groups
// (both the 32-bank/8-lane and the 64-bank/16-lane service patterns).  The
// 64-byte variant does the same for the int8 W8 weight rows.
__device__ __forceinline__ int swz128(int row) { return (row ^ (row >> 3)) & 7; }
__device__ __forceinline__ int swz64(int row) { return ((row >> 1) ^ (row >> 3)) & 3; }

__device__ __forceinline__ v4i buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

template <int MODE>
__device__ __forceinline__ typename ModeTraits<MODE>::Acc mfma32(v4i a, v4i b,
                                                                 typename ModeTraits<MODE>::Acc c) {
  if constexpr (MODE == GM_I8) return mfma32_i8(a, b, c);
  else if constexpr (MODE == GM_BF16) return mfma32_bf16(a, b, c);
  else return mfma32_f16(a, b, c);
}

__device__ __forceinline__ void store_out(void* c, int dt, int64_t idx, float v) {
  if (dt == DT_F16) reinterpret_cast<uint16_t*>(c)[idx] = f32_to_f16_bits(v);
  else if (dt == DT_BF16) reinterpret_cast<uint16_t*>(c)[idx] = f32_to_bf16(v);
  else reinterpret_cast<float*>(c)[idx] = v;
}
__device__ __forceinline__ float load_any(const void* p, int dt, int64_t idx) {
  if (dt == DT_F16) return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(p)[idx]);
  if (dt == DT_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[idx]);
  return reinterpret_cast<const float*>(p)[idx];
}

// Map a workgroup to its output tile.  Workgroup b runs on XCD b % 8; the
// renumbering makes the tiles of one XCD a contiguous run of `lin`, and the
// grouped order turns that run into a GROUP_M x k block of tiles.
__device__ __forceinline__ void tile_of(int tiles_m, int tiles_n, int& tm, int& tn) {
  const int ntiles = tiles_m * tiles_n;
  int lin = blockIdx.x;
  if ((ntiles & 7) == 0) lin = (blockIdx.x & 7) * (ntiles >> 3) + (blockIdx.x >> 3);
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_group = lin - group * per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One direct-to-LDS load: every lane fetches 16 bytes at voff + soff of the
// buffer and the wave's 64 results land contiguously (lane order) at `lds`
// (a wave-uniform address).  A plain function, not a template member: the
// builtin inside a kernel template stops the host pass from emitting the
// kernel's launch stub.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, char* lds, uint32_t voff,
                                      uint32_t soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr_t)lds, 16, voff, soff, 0, 0);
}

// vmcnt(0): this wave's direct-to-LDS loads have landed.
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }

template <int MODE, int BM, int BN, int WM, int WN, int EPI>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_kernel(GemmArgs p) {
  typedef ModeTraits<MODE> T;
  typedef typename T::Acc Acc;
  constexpr int NW = WM * WN;
  constexpr int NB = (EPI == GE_SWIGLU) ? 2 : 1;
  constexpr int A_BYTES = BM * 128;
  constexpr int B_BYTES = BN * T::BROW;
  constexpr int STAGE = A_BYTES + NB * B_BYTES;
  // 1 KiB direct-load blocks: 8 rows of a 128-byte row, or 16 of a 64-byte row
  constexpr int A_BLK = A_BYTES / 1024;
  constexpr int B_BLK = B_BYTES / 1024;
  constexpr int B_RPB = 1024 / T::BROW;
  constexpr int A_PER_W = A_BLK / NW;
  constexpr int B_PER_W = B_BLK / NW;
  static_assert(A_BLK % NW == 0 && B_BLK % NW == 0, "block split");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  static_assert(2 * STAGE <= 160 * 1024, "LDS budget");

  // Two stages as two distinct arrays: the compiler can then see that a
  // direct load into one stage never aliases the reads of the other.
  __shared__ __attribute__((aligned(1024))) char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) char st1[STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave index as a provably uniform (scalar) value: the direct-load LDS
  // address and scalar offset derive from it and must live in SGPRs
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int tiles_m = (int)((p.M + BM - 1) / BM);
  const int tiles_n = (int)((p.N + BN - 1) / BN);
  int tm, tn;
  tile_of(tiles_m, tiles_n, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t rows_a = min((int64_t)BM, p.M - m0);
  const int64_t rows_b = min((int64_t)BN, p.N - n0);
  const uint32_t lda_b = (uint32_t)(p.lda * T::EA);
  const uint32_t ldb_b = (uint32_t)(p.ldb * T::EB);
  const uint32_t ka_bytes = (uint32_t)(p.K * T::EA);

  __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const char*>(p.a) + m0 * lda_b), 0, (int)(rows_a * lda_b), 0x00020000);
  __amdgpu_buffer_rsrc_t rb[NB];
  rb[0] = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(reinterpret_cast<const char*>(p.b) + n0 * ldb_b), 0, (int)(rows_b * ldb_b), 0x00020000);
  if constexpr (NB == 2)
    rb[1] = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(reinterpret_cast<const char*>(p.b2) + n0 * ldb_b), 0, (int)(rows_b * ldb_b),
        0x00020000);

  // Direct-load addressing.  Lane L of a 1 KiB block fills physical chunk
  // L % cpr of block row L / cpr (cpr = 16-byte chunks per row) and fetches
  // the logical chunk the XOR swizzle maps there.  The block's first row is
  // a wave-uniform offset (the instruction's scalar offset); the lane part
  // is a row offset plus the swizzled chunk, recomputed per block from the
  // block index rather than kept in registers.
  const uint32_t a_lane_row = (uint32_t)(lane >> 3) * lda_b;
  const uint32_t b_lane_row = (uint32_t)(T::BROW == 128 ? (lane >> 3) : (lane >> 2)) * ldb_b;
  const int nk = (int)((p.K + T::BK - 1) / T::BK);
  const uint32_t kb_bytes = (uint32_t)(p.K * T::EB);

  // Enqueue the direct loads of K-stage kt into `st`.  Only the last stage
  // can overhang K; its chunks past K read as zero (offset out of range).
  auto dma_stage = [&](char* st, int kt) {
    const uint32_t ka = (uint32_t)kt * 128u;
    const uint32_t kb = (uint32_t)kt * T::BROW;
    const bool tail = ka + 128u > ka_bytes;
#pragma unroll
    for (int i = 0; i < A_PER_W; ++i) {
      const int blk = wave + i * NW;
      // row = 8*blk + lane/8, so swz128(row) = (lane/8 ^ blk) & 7
      const uint32_t kc = (uint32_t)(((lane & 7) ^ (lane >> 3) ^ blk) & 7) * 16u;
      uint32_t off = a_lane_row + kc + ka;
      if (tail && ka + kc >= ka_bytes) off = 0x80000000u;
      dma16(ra, st + blk * 1024, off, (uint32_t)blk * 8u * lda_b);
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int i = 0; i < B_PER_W; ++i) {
        const int blk = wave + i * NW;
        uint32_t kc;
        if constexpr (T::BROW == 128) {
          kc = (uint32_t)(((lane & 7) ^ (lane >> 3) ^ blk) & 7) * 16u;
        } else {
          const int row = blk * 16 + (lane >> 2);
          kc = (uint32_t)((lane & 3) ^ swz64(row)) * 16u;
        }
        uint32_t off = b_lane_row + kc + kb;
        if (tail && kb + kc >= kb_bytes) off = 0x80000000u;
        dma16(rb[nb], st + A_BYTES + nb * B_BYTES + blk * 1024, off,
              (uint32_t)blk * (uint32_t)B_RPB * ldb_b);
      }
  };

  Acc acc[NB][TM][TN];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[nb][i][j] = Acc{};

  const int lrow = lane & 31, lg = lane >> 5;

  auto compute = [&](const char* sa) {
    if constexpr (MODE != GM_W8) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        v4i af[TM];
        v4i bf[NB][TN];
        const int c = ks * 2 + lg;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          const int row = wm * WTM + i * 32 + lrow;
          af[i] = *reinterpret_cast<const v4i*>(sa + row * 128 + ((c ^ swz128(row)) << 4));
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int row = wn * WTN + j * 32 + lrow;
            bf[nb][j] = *reinterpret_cast<const v4i*>(sa + A_BYTES + nb * B_BYTES + row * 128 +
                                                      ((c ^ swz128(row)) << 4));
          }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[nb][i][j] = mfma32<MODE>(af[i], bf[nb][j], acc[nb][i][j]);
      }
    } else {
      // W8: a 16-byte int8 B read covers two MFMA k-steps.  Lane group g
      // supplies k = 32*jp + 16*g + 8*h + (0..7) in step h of pair jp, for
      // both operands, so every k of the stage is summed exactly once.
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        v4i bq[NB][TN];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            const int row = wn * WTN + j * 32 + lrow;
            const int c = 2 * jp + lg;
            bq[nb][j] = *reinterpret_cast<const v4i*>(sa + A_BYTES + nb * B_BYTES + row * 64 +
                                                      ((c ^ swz64(row)) << 4));
          }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          v4i af[TM];
          const int c = 4 * jp + 2 * lg + h;
#pragma unroll
          for (int i = 0; i < TM; ++i) {
            const int row = wm * WTM + i * 32 + lrow;
            af[i] = *reinterpret_cast<const v4i*>(sa + row * 128 + ((c ^ swz128(row)) << 4));
          }
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
              const v4i bw = __builtin_bit_cast(
                  v4i, i8x8_to_v8h((uint32_t)bq[nb][j][2 * h], (uint32_t)bq[nb][j][2 * h + 1]));
#pragma unroll
              for (int i = 0; i < TM; ++i) acc[nb][i][j] = mfma32_f16(af[i], bw, acc[nb][i][j]);
            }
        }
      }
    }
  };

  // Ping-pong over the two stages: the loads of stage k+1 are in flight
  // while stage k is consumed; one wait + barrier per stage.  The steady
  // state loop body is straight-line code (no conditional loads), so the
  // accumulators stay in one register class across iterations; the last one
  // or two stages are peeled after it.
  dma_stage(st0, 0);
  wait_dma();
  __syncthreads();
  // sched_barrier(0) pins each stage's load issue ahead of the MFMA block;
  // left alone, the scheduler sinks the loads to just before the wait,
  // which serializes load latency with compute.
  int kt = 0;
  for (; kt + 2 < nk; kt += 2) {
    dma_stage(st1, kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(st0);
    wait_dma();
    __syncthreads();
    dma_stage(st0, kt + 2);
    __builtin_amdgcn_sched_barrier(0);
    compute(st1);
    wait_dma();
    __syncthreads();
  }
  if (kt + 1 < nk) {
    dma_stage(st1, kt + 1);
    __builtin_amdgcn_sched_barrier(0);
    compute(st0);
    wait_dma();
    __syncthreads();
    compute(st1);
  } else {
    compute(st0);
  }

  // ---- epilogue ----------------------------------------------------------
  // Lane (lrow, lg) of sub-tile (i, j) holds column lrow and rows
  // 8*(r/4) + 4*lg + (r%4) in accumulator register r.  All loops are
  // compile-time (static_for), so the accumulators never leave registers;
  // per-column scales are loaded once per sub-tile column, per-row scales
  // once per sub-tile row.
  const int64_t row_base = m0 + wm * WTM + 4 * lg;
  const int64_t col_base = n0 + wn * WTN + lrow;
  float cs[TN], cs2[TN];
  static_for<TN>([&](auto jc) {
    constexpr int j = decltype(jc)::value;
    const int64_t col = col_base + j * 32;
    cs[j] = (p.col_scale && col < p.N) ? p.col_scale[col] : 1.f;
    cs2[j] = (NB == 2 && p.col_scale2 && col < p.N) ? p.col_scale2[col] : 1.f;
  });
  const int odt = p.out_dtype;
  static_for<TM>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    float rs[16];
    static_for<16>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      const int64_t row = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
      rs[r] = (MODE == GM_I8 && p.row_scale && row < p.M) ? p.row_scale[row] : 1.f;
    });
    static_for<TN>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      const int64_t col = col_base + j * 32;
      if (col < p.N) {
        static_for<16>([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          const int64_t row = row_base + i * 32 + 8 * (r >> 2) + (r & 3);
          if (row < p.M) {
            const int64_t idx = row * p.ldc + col;
            if constexpr (MODE == GM_I8) {
              const int v = acc[0][i][j][r];
              if (odt == DT_I32) {
                reinterpret_cast<int*>(p.c)[idx] = v;
              } else {
                float t = (float)v;
                if (p.row_scale) t = t * rs[r];
                if (p.col_scale) t = t * cs[j];
                store_out(p.c, odt, idx, t);
              }
            } else if constexpr (EPI == GE_SWIGLU) {
              const float g = f16_bits_to_f32(f32_to_f16_bits(acc[0][i][j][r] * cs[j]));
              const float u = f16_bits_to_f32(f32_to_f16_bits(acc[NB - 1][i][j][r] * cs2[j]));
              const float sg = g / (1.0f + fast_exp(-g));
              reinterpret_cast<uint16_t*>(p.c)[idx] = f32_to_f16_bits(sg * u);
            } else {
              float t = acc[0][i][j][r];
              if (p.col_scale) t = t * cs[j];
              if (p.res) t = t + load_any(p.res, p.res_dtype, row * p.ldr + col);
              store_out(p.c, odt, idx, t);
            }
          }
        });
      }
    });
  });
}

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

// ---------------------------------------------------------------------------
// Config table.  The autotuner searches over these instantiations.
// ---------------------------------------------------------------------------
typedef void (*GemmLaunch)(const GemmArgs&, hipStream_t);

template <int MODE, int BM, int BN, int WM, int WN, int EPI>
static void launch_one(const GemmArgs& a, hipStream_t s) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  gemm_kernel<MODE, BM, BN, WM, WN, EPI><<<dim3((unsigned)tiles), dim3(64 * WM * WN), 0, s>>>(a);
}

struct GemmEntry {
  GemmConfig cfg;
  GemmLaunch fn;
};

#define HX_GEMM_CFGS(MODE)                                                                 \
  {{256, 256, 2, 2, GE_STORE, "256x256_w2x2"}, &launch_one<MODE, 256, 256, 2, 2, GE_STORE>}, \
  {{256, 128, 2, 2, GE_STORE, "256x128_w2x2"}, &launch_one<MODE, 256, 128, 2, 2, GE_STORE>}, \
  {{128, 256, 2, 2, GE_STORE, "128x256_w2x2"}, &launch_one<MODE, 128, 256, 2, 2, GE_STORE>}, \
  {{128, 128, 2, 2, GE_STORE, "128x128_w2x2"}, &launch_one<MODE, 128, 128, 2, 2, GE_STORE>}, \
  {{256, 256, 2, 4, GE_STORE, "256x256_w2x4"}, &launch_one<MODE, 256, 256, 2, 4, GE_STORE>}, \
  {{64, 64, 2, 2, GE_STORE, "64x64_w2x2"}, &launch_one<MODE, 64, 64, 2, 2, GE_STORE>}

static const GemmEntry kI8[] = {HX_GEMM_CFGS(GM_I8)};
static const GemmEntry kF16[] = {HX_GEMM_CFGS(GM_F16)};
static const GemmEntry kBF16[] = {HX_GEMM_CFGS(GM_BF16)};
static const GemmEntry kW8[] = {
    HX_GEMM_CFGS(GM_W8),
    {{256, 128, 2, 2, GE_SWIGLU, "swiglu_256x128_w2x2"}, &launch_one<GM_W8, 256, 128, 2, 2, GE_SWIGLU>},
    {{128, 128, 2, 2, GE_SWIGLU, "swiglu_128x128_w2x2"}, &launch_one<GM_W8, 128, 128, 2, 2, GE_SWIGLU>},
    {{128, 64, 2, 2, GE_SWIGLU, "swiglu_128x64_w2x2"}, &launch_one<GM_W8, 128, 64, 2, 2, GE_SWIGLU>},
};

static const GemmEntry* table(int mode, int& n) {
  switch (mode) {
    case GM_I8: n = (int)(sizeof(kI8) / sizeof(kI8[0])); return kI8;
    case GM_F16: n = (int)(sizeof(kF16) / sizeof(kF16[0])); return kF16;
    case GM_BF16: n = (int)(sizeof(kBF16) / sizeof(kBF16[0])); return kBF16;
    case GM_W8: n = (int)(sizeof(kW8) / sizeof(kW8[0])); return kW8;
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

static int g_num_cus = 0;
static int num_cus() {
  if (g_num_cus == 0) {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      g_num_cus = v;
    else
      g_num_cus = 256;
  }
  return g_num_cus;
}

// Untuned choice: estimated time = waves_of_tiles * tile_area / efficiency.
// The efficiencies are relative throughputs measured on MI355X at 4096^3
// (the 8-wave 256x256 tile is the fastest per MAC; 128x128 beats the
// 4-wave 256-wide tiles); the autotuner replaces this guess per shape.
int gemm_default_config(int mode, int epi, int64_t M, int64_t N, int64_t K) {
  (void)K;
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t) return -1;
  const int cus = num_cus();
  int best = -1;
  double best_cost = 0;
  for (int i = 0; i < n; ++i) {
    const GemmConfig& c = t[i].cfg;
    if (c.epi != epi) continue;
    const double tiles = (double)((M + c.bm - 1) / c.bm) * (double)((N + c.bn - 1) / c.bn);
    const double waves = (double)(int64_t)((tiles + cus - 1) / cus);
    const double area = (double)c.bm * c.bn;
    double eff;
    if (area >= 65536) eff = (c.wm * c.wn == 8) ? 1.0 : 0.72;
    else if (area >= 32768) eff = 0.68;
    else if (area >= 16384) eff = 0.78;
    else eff = 0.55;
    const double cost = waves * area / eff;
    if (best < 0 || cost < best_cost - 1e-9) {
      best = i;
      best_cost = cost;
    }
  }
  return best;
}

bool gemm_fast_ok(int mode, const GemmArgs& a) {
  const int ea = (mode == GM_I8) ? 1 : 2;
  const int eb = (mode == GM_I8 || mode == GM_W8) ? 1 : 2;
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (!al16(a.a) || !al16(a.b) || (a.b2 && !al16(a.b2))) return false;
  if ((a.lda * ea) % 16 != 0 || (a.ldb * eb) % 16 != 0) return false;
  if ((a.K * ea) % 16 != 0 || (a.K * eb) % 16 != 0) return false;
  // 32-bit buffer offsets inside one tile's row range
  if ((int64_t)256 * a.lda * ea >= ((int64_t)1 << 31)) return false;
  if ((int64_t)256 * a.ldb * eb >= ((int64_t)1 << 31)) return false;
  if (a.M <= 0 || a.N <= 0 || a.K <= 0) return false;
  return true;
}

int launch_gemm(int mode, int cfg_idx, const GemmArgs& a, hipStream_t s) {
  int n;
  const GemmEntry* t = table(mode, n);
  if (!t || cfg_idx < 0 || cfg_idx >= n) return HXI_ERR_ARG;
  const int64_t tiles = ((a.M + t[cfg_idx].cfg.bm - 1) / t[cfg_idx].cfg.bm) *
                        ((a.N + t[cfg_idx].cfg.bn - 1) / t[cfg_idx].cfg.bn);
  if (tiles <= 0 || tiles > 0x7fffffff) return HXI_ERR_SHAPE;
  t[cfg_idx].fn(a, s);
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
