// hx_gemm_kernel.hpp -- MFMA GEMM family for gfx950: int8 x int8 -> int32,
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
//     accumulators stay in registers for the whole K loop;
//   * K is walked in stages of 128 bytes of A per row, double-buffered in
//     LDS; each stage is fetched with direct-to-LDS 16-byte buffer loads
//     (rows past the matrix edge and the K tail read as zero from the buffer
//     descriptor's range), one LDS-only barrier per stage;
//   * LDS rows are 128 (or 64) bytes with the 16-byte chunk index XOR-swizzled
//     by the row so that the MFMA operand reads (16 bytes per lane, 32 rows)
//     and the stage writes are bank-conflict free;
//   * operand fragments are double-buffered in registers (the reads of k-step
//     s+1 are in flight while the MFMAs of step s run);
//   * B is consumed K-contiguous ([N][K]), i.e. the weight image the resident
//     registry keeps -- the counterpart of the reference's pre-packed WH
//     crouton image (QHB/backend/hmx_weight_prepack.py:171-212);
//   * the epilogue converts each wave's block in LDS and writes whole rows;
//   * workgroup ids are renumbered so that each XCD (workgroups are dealt to
//     the 8 XCDs round robin) walks a compact block of tiles: the B strips of
//     that block stay resident in the XCD's L2 while its M-tiles go by.
#pragma once

#include "hx_device.hpp"
#include "hx_internal.hpp"
#include <type_traits>

namespace hx {

template <int MODE> struct ModeTraits;
template <> struct ModeTraits<GM_I8> {
  static constexpr int EA = 1, EB = 1;  // operand element bytes
  typedef v16i Acc;
};
template <> struct ModeTraits<GM_F16> {
  static constexpr int EA = 2, EB = 2;
  typedef v16f Acc;
};
template <> struct ModeTraits<GM_BF16> {
  static constexpr int EA = 2, EB = 2;
  typedef v16f Acc;
};
template <> struct ModeTraits<GM_W8> {
  static constexpr int EA = 2, EB = 1, BK = 64, BROW = 64;
  typedef v16f Acc;
};

// Chunk swizzles.  For 128-byte rows, (row ^ row>>3) & 7 makes any 8 and any
// 16 consecutive rows reading the same logical chunk hit distinct bank groups
// (both the 32-bank/8-lane and the 64-bank/16-lane service patterns).
__device__ __forceinline__ int swz128(int row) { return (row ^ (row >> 3)) & 7; }

// 64-byte rows (the W8 weight tile, 64-byte int8 stages): the chunk is XORed
// with the row's index among groups of four.  Timed on the fragment read
// pattern (32 rows x 2 adjacent chunks per wave read): 2.08 ns per wave read
// per CU, against 3.52 for ((row >> 1) ^ (row >> 3)) & 3 and 6.75 unswizzled
// (the 128-byte rows' swz128: 2.38).
__device__ __forceinline__ int swz64(int row) { return (row >> 2) & 3; }
// 256-byte rows: 16 consecutive rows (one 16-lane service group of a
// 16-byte read) reading the same logical chunk cover all 16 chunk slots.
__device__ __forceinline__ int swz256(int row) { return (row ^ (row >> 4)) & 15; }
template <int RB>
__device__ __forceinline__ int swz_rows(int row) {
  if constexpr (RB == 256) return swz256(row);
  else if constexpr (RB == 128) return swz128(row);
  else return swz64(row);
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

// The grouped order: linear tile number -> tile, walking GROUP_M M-tiles of
// one B strip, then the same M-tiles of the next strip, so a contiguous
// run of numbers covers a GROUP_M x k block of tiles (its A and B strips
// stay in one XCD's L2 while the block goes by).
__device__ __forceinline__ void tile_of_lin(int lin, int tiles_m, int tiles_n, int& tm, int& tn) {
  constexpr int GROUP_M = 4;
  const int per_group = GROUP_M * tiles_n;
  const int group = lin / per_group;
  const int first_m = group * GROUP_M;
  const int gm = min(tiles_m - first_m, GROUP_M);
  const int in_group = lin - group * per_group;
  tm = first_m + in_group % gm;
  tn = in_group / gm;
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

__device__ __forceinline__ v4f load4(const void* p, int dt, int64_t idx) {
  if (dt == DT_F32) return *reinterpret_cast<const v4f*>(reinterpret_cast<const float*>(p) + idx);
  const v2i w = *reinterpret_cast<const v2i*>(reinterpret_cast<const uint16_t*>(p) + idx);
  const uint32_t lo = (uint32_t)w[0], hi = (uint32_t)w[1];
  if (dt == DT_F16)
    return v4f{f16_bits_to_f32((uint16_t)lo), f16_bits_to_f32((uint16_t)(lo >> 16)),
               f16_bits_to_f32((uint16_t)hi), f16_bits_to_f32((uint16_t)(hi >> 16))};
  return v4f{bf16_to_f32((uint16_t)lo), bf16_to_f32((uint16_t)(lo >> 16)), bf16_to_f32((uint16_t)hi),
             bf16_to_f32((uint16_t)(hi >> 16))};
}

// Scheduling recipe of one k-step: its NMF MFMAs, each followed by one of
// the NREAD LDS reads of the next step (while any remain) and its share of
// the NVM direct loads.  Reads issued as one burst ahead of the MFMAs queue
// behind every other wave's burst on the LDS; spread between the MFMAs they
// arrive in time for the next step (measured at 4096^3 int8: 59.6 against
// 60.5 us, 110.9 against 112.9 at K = 8192).
template <int NREAD, int NMF, int NVM>
__device__ __forceinline__ void interleave_reads_mfma_vmem() {
  constexpr int PER = (NVM + NMF - 1) / NMF;  // loads after each MFMA
  static_for<NMF>([](auto ic) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // one MFMA
    if constexpr (decltype(ic)::value < NREAD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // a DS read
    if constexpr (PER > 0) __builtin_amdgcn_sched_group_barrier(0x020, PER, 0);  // its share of the direct loads
  });
}

// SB: bytes of A per row in one K stage (64, 128 or 256; the W8 mode takes
// 128 only).  Smaller stages cut the LDS a workgroup holds
// (more workgroups per CU, or a third stage), larger ones halve the
// barriers per K.  STAGES: K stages held in LDS at once (2: double buffer,
// 3: the loads of stage kt+2 are in flight while stage kt is consumed).
// MINW: waves per SIMD the register budget must allow (2 caps a wave at 256
// registers).
// BKN (f16 / bf16): B is [K][N], N contiguous.  A stage then holds BKE rows
// of k, each BN elements, with 64-byte segments XOR-swizzled by the row; the
// B operand of each MFMA step comes from two transposing LDS reads
// (ds_read_b64_tr_b16: within each 16-lane group, lane 4a+b receives
// element b of the 8-byte chunks addressed by lanes a, a+4, a+8, a+12), so
// lane l = 16G + i, addressing row 16ks + 8(G/2) + 4h + i/4 at column
// 16(G%2) + 4(i%4) of its 32-column sub-tile, receives column l % 32 at
// k = 16ks + 8(l/32) + 4h + (0..3) -- the K-contiguous operand without a
// transpose of B in memory.
// BKN int8: the same with ds_read_b64_tr_b8 (within each 16-lane group,
// lane 8a+b receives element b of the 8-byte chunks addressed by lanes a,
// a+2, ..., a+14) and the 16-byte chunks of a k row XOR-swizzled so that the
// 8 consecutive rows x 2 adjacent chunks that a half-wave reads cover 16
// distinct bank groups: lane
// l = 16G + i, addressing row 32ks + 16(G/2) + 8h + i/2 at column
// 16(G%2) + 8(i%2) of its 32-column sub-tile, receives column l % 32 at
// k = 32ks + 16(l/32) + 8h + (0..7).
//
// PERSIST: one workgroup per CU walks a run of consecutive M-tiles of one B
// strip (the weight strip stays hot while its M-tiles go by) and overlaps
// each tile's epilogue with the next tile's first K stages: after the last
// K stage the next tile's stage loads are issued first, then the finished
// tile is converted and stored through a staging region of its own, so its
// stores drain while the next tile's loads land and its first MFMAs run.
// Interior shapes only (no EDGE), B as [N][K], 16-bit outputs.
//
// SPLITM: the K split's parts merge inside the kernel (p.cnt, p.part) -- a
// compile-time variant, so the other kernels carry none of its code.
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int SB = 128, int MINW = 1, bool EDGE = false,
          bool BKN = false, int STAGES = 2, bool PERSIST = false, bool SPLITM = false>
__global__ void __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(MINW, 8)))
gemm_kernel(GemmArgs p) {
  typedef ModeTraits<MODE> T;
  typedef typename T::Acc Acc;
  static_assert(SB == 128 || ((SB == 64 || SB == 256) && MODE != GM_W8), "stage width");
  static_assert(STAGES == 2 || STAGES == 3, "stage count");
  static_assert(!BKN || ((MODE == GM_F16 || MODE == GM_BF16 || MODE == GM_I8) && EPI == GE_STORE), "[K][N] B");
  constexpr int NW = WM * WN;
  constexpr int NB = (EPI == GE_SWIGLU) ? 2 : 1;
  constexpr int BROW = (MODE == GM_W8) ? SB / 2 : SB;  // bytes of B per row in one stage
  constexpr int KSTEPS = SB / 32;                      // MFMA k-steps per stage
  constexpr int A_BYTES = BM * SB;
  constexpr int B_BYTES = BN * BROW;
  constexpr int STAGE = A_BYTES + NB * B_BYTES;
  // 1 KiB direct-load blocks: 8 rows of a 128-byte row, or 16 of a 64-byte row
  constexpr int A_BLK = A_BYTES / 1024;
  constexpr int B_BLK = B_BYTES / 1024;
  constexpr int A_RPB = 1024 / SB;
  constexpr int B_RPB = 1024 / BROW;
  constexpr int A_CPR = SB / 16, B_CPR = BROW / 16;  // 16-byte chunks per row
  constexpr int A_PER_W = A_BLK / NW;
  constexpr int B_PER_W = B_BLK / NW;
  constexpr int P = A_PER_W + NB * B_PER_W;  // direct loads per wave per stage
  static_assert(A_BLK % NW == 0 && B_BLK % NW == 0, "block split");
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WTM % 32 == 0 && WTN % 32 == 0, "wave tile");
  // per-row / per-column scales of this tile, fetched in the prologue
  // (SC_ROWS floats each: one 1 KiB direct load covers 256)
  constexpr int SC_ROWS = (BM > BN ? BM : BN) < 256 ? 256 : (BM > BN ? BM : BN);
  // PERSIST: the scales of two tiles (the finished one's epilogue reads its
  // set while the next tile's set is loading) and a staging region of 32
  // rows x WTN 16-bit outputs per wave, apart from the stage buffers
  constexpr int SC_SETS = PERSIST ? 2 : 1;
  constexpr int STG_WAVE = 32 * WTN * 2;
  constexpr int STG = PERSIST ? NW * STG_WAVE : 16;
  static_assert(!PERSIST || (!EDGE && !BKN), "persistent: interior shapes, B as [N][K]");
  static_assert(!(PERSIST && SPLITM), "persistent configs do not split K");
  static_assert(STAGES * STAGE + SC_SETS * (1 + NB) * SC_ROWS * 4 + (PERSIST ? STG : 0) <= 160 * 1024,
                "LDS budget");
  static_assert(STAGES * P < 64, "vmcnt range");

  // The stages as distinct arrays: the compiler can then see that a direct
  // load into one stage never aliases the reads of another.
  __shared__ __attribute__((aligned(1024))) char st0[STAGE];
  __shared__ __attribute__((aligned(1024))) float scl_all[SC_SETS * (1 + NB) * SC_ROWS];
  __shared__ __attribute__((aligned(1024))) char st1[STAGE];
  __shared__ __attribute__((aligned(1024))) char st2[STAGES == 3 ? STAGE : 16];
  __shared__ __attribute__((aligned(1024))) char stg[STG];
  __shared__ int is_last_part;

  // measurement hook: this workgroup's shader-clock cycles and
  // constant-rate ticks, added to p.clk when it ends
  uint64_t clk_c0 = 0, clk_r0 = 0;
  if (p.clk) {
    clk_c0 = __builtin_amdgcn_s_memtime();
    clk_r0 = __builtin_amdgcn_s_memrealtime();
  }
  auto clock_out = [&]() __attribute__((always_inline)) {
    if (p.clk && threadIdx.x == 0) {
      const uint64_t c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
      atomicAdd(p.clk, (unsigned long long)(c1 - clk_c0));
      atomicAdd(p.clk + 1, (unsigned long long)(r1 - clk_r0));
      atomicAdd(p.clk + 2, 1ull);
    }
  };

  // K split: workgroup row blockIdx.y sums k in [y k_split, (y+1) k_split).
  // With counters (merge_in) the parts of a tile hand their partials to the
  // last of them to finish, which runs the epilogue; without, part y writes
  // the binary32 slice y of c and launch_gemm merges the slices.
  constexpr bool merge_in = SPLITM;
  if (gridDim.y > 1) {
    const int64_t k0 = (int64_t)blockIdx.y * p.k_split;
    p.a = reinterpret_cast<const char*>(p.a) + k0 * T::EA;
    p.b = reinterpret_cast<const char*>(p.b) + k0 * (BKN ? p.ldb : 1) * T::EB;
    p.K = min(p.k_split, p.K - k0);
    if (!merge_in) p.c = reinterpret_cast<char*>(p.c) + (int64_t)blockIdx.y * p.M * p.ldc * 4;
  }

  const int tid = threadIdx.x;
  // lane and wave: a persistent workgroup passes them through an empty asm
  // at the start of every tile, so what derives from them is recomputed per
  // tile instead of being held across the K loop
  int lane = tid & 63;
  // wave index as a provably uniform (scalar) value: the direct-load LDS
  // address and scalar offset derive from it and must live in SGPRs
  int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tiles_m = (int)((p.M + BM - 1) / BM);
  const int tiles_n = (int)((p.N + BN - 1) / BN);
  const uint32_t lda_b = (uint32_t)(p.lda * T::EA);
  const uint32_t ldb_b = (uint32_t)(p.ldb * T::EB);
  const uint32_t ka_bytes = (uint32_t)(p.K * T::EA);

  // Per-tile state: coordinates, rows in range, buffer descriptors.
  int tm = 0, tn = 0;
  int64_t m0 = 0, n0 = 0, rows_a = 0, rows_b = 0;
  __amdgpu_buffer_rsrc_t ra;
  __amdgpu_buffer_rsrc_t rb[NB];
  auto set_tile = [&](int tm_, int tn_) __attribute__((always_inline)) {
    // The tile coordinates are workgroup-uniform, but integer divisions run
    // on the vector ALU; readfirstlane states the uniformity, so the buffer
    // descriptors built from them stay scalar (a descriptor the compiler
    // believes divergent turns every buffer load into a loop over lanes).
    tm = __builtin_amdgcn_readfirstlane(tm_);
    tn = __builtin_amdgcn_readfirstlane(tn_);
    m0 = (int64_t)tm * BM;
    n0 = (int64_t)tn * BN;
    rows_a = min((int64_t)BM, p.M - m0);
    rows_b = min((int64_t)BN, p.N - n0);
    ra = __builtin_amdgcn_make_buffer_rsrc((void*)(reinterpret_cast<const char*>(p.a) + m0 * lda_b), 0,
                                           (int)(rows_a * lda_b), 0x00020000);
    if constexpr (BKN) {
      // columns n0.. of every row of k, up to the matrix's last element
      rb[0] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(reinterpret_cast<const char*>(p.b) + n0 * T::EB), 0,
          (int)(((p.K - 1) * p.ldb + (p.N - n0)) * T::EB), 0x00020000);
    } else {
      rb[0] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(reinterpret_cast<const char*>(p.b) + n0 * ldb_b), 0, (int)(rows_b * ldb_b), 0x00020000);
    }
    if constexpr (NB == 2)
      rb[1] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(reinterpret_cast<const char*>(p.b2) + n0 * ldb_b), 0, (int)(rows_b * ldb_b),
          0x00020000);
  };
  // PERSIST: this workgroup's run of tiles.  Tiles are numbered in the
  // grouped order (consecutive numbers are consecutive M-tiles of one B
  // strip, GROUP_M at a time) and cut into gridDim.x runs whose lengths
  // differ by at most one; workgroup b runs on XCD b % 8, so the runs are
  // renumbered to give each XCD a contiguous range of numbers -- a compact
  // block of tiles whose A and B strips its L2 holds.
  int t_cur = 0, t_end = 0;
  if constexpr (PERSIST) {
    const int ntiles = tiles_m * tiles_n;
    const int G = gridDim.x;
    int w = blockIdx.x;
    if ((G & 7) == 0) w = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);
    t_cur = __builtin_amdgcn_readfirstlane((int)((int64_t)w * ntiles / G));
    t_end = __builtin_amdgcn_readfirstlane((int)((int64_t)(w + 1) * ntiles / G));
    int tm_, tn_;
    tile_of_lin(t_cur, tiles_m, tiles_n, tm_, tn_);
    set_tile(tm_, tn_);
  } else {
    int tm_, tn_;
    tile_of(tiles_m, tiles_n, tm_, tn_);
    set_tile(tm_, tn_);
  }
  int wm = wave / WN, wn = wave % WN;

  // Direct-load addressing.  Lane L of a 1 KiB block fills physical chunk
  // L % cpr of block row L / cpr (cpr = 16-byte chunks per row) and fetches
  // the logical chunk the XOR swizzle maps there.  The block's first row is
  // a wave-uniform offset (the instruction's scalar offset); the lane part
  // is a row offset plus the swizzled chunk, recomputed per block from the
  // block index rather than kept in registers.
  // EDGE (M or N not a multiple of the tile): lanes whose row lies past the
  // tile's last row get an out-of-range vector offset.  The block's row
  // offset travels in the scalar offset, and the zero fill must not depend
  // on whether the range check includes it.  Block blk's lane row is past
  // the edge when blk * RPB >= lim.  Interior shapes skip the test (it costs
  // ~1% at 4096^3).
  constexpr int BKE = SB / T::EA;  // elements of K per stage
  // BKN stage layout: BKE rows of k, KROWB bytes each, 64-byte segments
  // XOR-swizzled so that the 8 rows one transposing read touches (4 + 4,
  // 8 apart) spread over the four 64-byte bank groups
  constexpr int KROWB = BN * T::EB;
  constexpr int KCPR = KROWB / 16;
  constexpr int KRPB = KROWB >= 1024 ? 1 : 1024 / KROWB;
  constexpr int KNSEG = KROWB / 64;
  auto swz_kn = [](int row) -> int {
    if constexpr (KNSEG >= 4) return row & 3;
    else if constexpr (KNSEG == 2) return (row >> 1) & 1;
    else return 0;
  };
  // int8: 16-byte chunks, KRW rows per 256-byte bank window; the chunk is
  // XORed with twice the row's window index among 8 consecutive rows, so an
  // even chunk and its odd neighbour (read together) never collide
  constexpr int KRW = KCPR >= 16 ? 1 : 16 / KCPR;
  auto swz_kn8 = [](int row) -> int { return ((row / KRW) & (8 / KRW - 1)) << 1; };
  const int nk = (int)((p.K + BKE - 1) / BKE);
  const uint32_t kb_bytes = (uint32_t)(p.K * T::EB);

  // Enqueue the direct loads of K-stage kt into `st`.  Only the last stage
  // can overhang K; its chunks past K read as zero (offset out of range).
  // MASK = false is for stages known not to be the last one.
  auto dma_stage = [&](char* st, int kt, auto maskc) __attribute__((always_inline)) {
    constexpr bool MASK = decltype(maskc)::value;
    const uint32_t a_lane_row = (uint32_t)(lane / A_CPR) * lda_b;
    const uint32_t b_lane_row = (uint32_t)(lane / B_CPR) * ldb_b;
    const int a_lim = (int)rows_a - lane / A_CPR;
    const int b_lim = (int)rows_b - lane / B_CPR;
    const uint32_t ka = (uint32_t)kt * (uint32_t)SB;
    const uint32_t kb = (uint32_t)kt * (uint32_t)BROW;
    const bool tail = MASK && ka + (uint32_t)SB > ka_bytes;
    static_for<A_PER_W>([&](auto ic) {
      const int blk = wave + decltype(ic)::value * NW;
      uint32_t kc;
      if constexpr (SB == 128) {
        // row = 8*blk + lane/8, so swz128(row) = (lane/8 ^ blk) & 7
        kc = (uint32_t)(((lane & 7) ^ (lane >> 3) ^ blk) & 7) * 16u;
      } else {
        const int row = blk * A_RPB + lane / A_CPR;
        kc = (uint32_t)((lane % A_CPR) ^ swz_rows<SB>(row)) * 16u;
      }
      uint32_t off = a_lane_row + kc + ka;
      if (tail && ka + kc >= ka_bytes) off = 0x80000000u;
      if constexpr (EDGE)
        if (blk * A_RPB >= a_lim) off = 0x80000000u;
      dma16(ra, st + blk * 1024, off, (uint32_t)blk * (uint32_t)A_RPB * lda_b);
    });
    if constexpr (BKN) {
      // block blk holds k rows blk*KRPB .. of the stage, 16-byte chunk
      // lane % KCPR of row lane / KCPR; the lane fetches the logical
      // segment the row's swizzle maps to its physical one
      static_for<B_PER_W>([&](auto ic) {
        const int blk = wave + decltype(ic)::value * NW;
        const int row = blk * KRPB + lane / KCPR, pc = lane % KCPR;
        const int lcol = MODE == GM_I8 ? (pc ^ swz_kn8(row))                    // logical chunk
                                       : ((((pc >> 2) ^ swz_kn(row)) << 2) | (pc & 3));
        const uint32_t k = (uint32_t)kt * (uint32_t)BKE + (uint32_t)row;
        uint32_t off = k * ldb_b + (uint32_t)lcol * 16u;
        if (k >= (uint32_t)p.K) off = 0x80000000u;
        dma16(rb[0], st + A_BYTES + blk * 1024, off, 0u);
      });
      return;
    }
    static_for<NB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      static_for<B_PER_W>([&](auto ic) {
        const int blk = wave + decltype(ic)::value * NW;
        uint32_t kc;
        if constexpr (BROW == 128) {
          kc = (uint32_t)(((lane & 7) ^ (lane >> 3) ^ blk) & 7) * 16u;
        } else {
          const int row = blk * B_RPB + lane / B_CPR;
          kc = (uint32_t)((lane % B_CPR) ^ swz_rows<BROW>(row)) * 16u;
        }
        uint32_t off = b_lane_row + kc + kb;
        if (tail && kb + kc >= kb_bytes) off = 0x80000000u;
        if constexpr (EDGE)
          if (blk * B_RPB >= b_lim) off = 0x80000000u;
        dma16(rb[nb], st + A_BYTES + nb * B_BYTES + blk * 1024, off,
              (uint32_t)blk * (uint32_t)B_RPB * ldb_b);
      });
    });
  };

  Acc acc[NB][TM][TN];
  static_for<NB>([&](auto nbc) {
    static_for<TM>([&](auto ic) {
      static_for<TN>([&](auto jc) {
        acc[decltype(nbc)::value][decltype(ic)::value][decltype(jc)::value] = Acc{};
      });
    });
  });

  int lrow = lane & 31, lg = lane >> 5;

  // Operand fragments, double-buffered in registers: while the MFMAs of
  // k-step ks run, the LDS reads of step ks+1 are in flight.  A stage is
  // KSTEPS k-steps.  For W8 one 16-byte int8 B read covers two steps (it is widened
  // to f16 half by half), so B is read on even steps into its own pair of
  // buffers, indexed by the step pair.
  v4i fa[2][TM];
  v4i fb[2][NB][TN];

  auto read_frags = [&](const char* sa, auto ksc) __attribute__((always_inline)) {
    constexpr int ks = decltype(ksc)::value;
    constexpr int s = ks & 1;
    typedef short v4s_t __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) v4s_t* lds_v4s_t;
    // step ks reads A chunk ca (W8: A is f16, step ks = 2*jp + h covers
    // k = 32*jp + 16*g + 8*h + (0..7) for lane group g, both operands, so
    // every k of the stage is summed exactly once)
    const int ca = (MODE != GM_W8) ? ks * 2 + lg : 4 * (ks >> 1) + 2 * lg + (ks & 1);
    auto swz = [](int row) -> int { return swz_rows<SB>(row); };
    static_for<TM>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      const int row = wm * WTM + i * 32 + lrow;
      fa[s][i] = *reinterpret_cast<const v4i*>(sa + row * SB + ((ca ^ swz(row)) << 4));
    });
    if constexpr (BKN && MODE == GM_I8) {
      const int G = lane >> 4, i = lane & 15;
      typedef __attribute__((address_space(3))) v2i* lds_v2i_t;
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int colb = wn * WTN + 32 * j + 16 * (G & 1) + 8 * (i & 1);  // byte (column) in the row
        v2i hv[2];
        static_for<2>([&](auto hc) {
          constexpr int h = decltype(hc)::value;
          const int row = 32 * ks + 16 * (G >> 1) + 8 * h + (i >> 1);
          const char* a = sa + A_BYTES + row * KROWB + (((colb >> 4) ^ swz_kn8(row)) << 4) + (colb & 15);
          hv[h] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t)a);
        });
        fb[s][0][j] = v4i{hv[0][0], hv[0][1], hv[1][0], hv[1][1]};
      });
    } else if constexpr (BKN) {
      const int G = lane >> 4, i = lane & 15;
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int colb = (wn * WTN + 32 * j + 16 * (G & 1) + 4 * (i & 3)) * T::EB;  // byte in the row
        v2i hv[2];
        static_for<2>([&](auto hc) {
          constexpr int h = decltype(hc)::value;
          const int row = 16 * ks + 8 * (G >> 1) + 4 * h + (i >> 2);
          const char* a = sa + A_BYTES + row * KROWB + (((colb >> 6) ^ swz_kn(row)) << 6) + (colb & 63);
          hv[h] = __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t)a));
        });
        fb[s][0][j] = v4i{hv[0][0], hv[0][1], hv[1][0], hv[1][1]};
      });
    } else if constexpr (MODE != GM_W8) {
      static_for<NB>([&](auto nbc) {
        constexpr int nb = decltype(nbc)::value;
        static_for<TN>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          const int row = wn * WTN + j * 32 + lrow;
          fb[s][nb][j] = *reinterpret_cast<const v4i*>(sa + A_BYTES + nb * B_BYTES + row * SB +
                                                       ((ca ^ swz(row)) << 4));
        });
      });
    } else if constexpr ((ks & 1) == 0) {
      constexpr int jp = ks >> 1;
      const int cb = 2 * jp + lg;
      static_for<NB>([&](auto nbc) {
        constexpr int nb = decltype(nbc)::value;
        static_for<TN>([&](auto jc) {
          constexpr int j = decltype(jc)::value;
          const int row = wn * WTN + j * 32 + lrow;
          fb[jp][nb][j] = *reinterpret_cast<const v4i*>(sa + A_BYTES + nb * B_BYTES + row * 64 +
                                                        ((cb ^ swz64(row)) << 4));
        });
      });
    }
  };

  // The MFMAs of one k-step.  B is the first operand, so the accumulators
  // hold C transposed: lane (lrow, lg) of sub-tile (i, j) holds row lrow and
  // the four consecutive columns 8*g + 4*lg + (0..3) in registers 4g..4g+3.
  // Order (int8 / f16 / bf16): the A fragment fixed across the TN MFMAs of
  // a row of sub-tiles, the B fragments walked back and forth so each row
  // starts with the B fragment the previous one ended with (measured at
  // 4096^3 int8, interleaved in one process: 58.5 against 59.1 us on random
  // operands, 40.1 against 40.8 on zeros, against B fixed and A walked).
  // W8 widens each B fragment once per k-step and keeps B fixed instead.
  auto mfmas = [&](auto ksc) __attribute__((always_inline)) {
    constexpr int ks = decltype(ksc)::value;
    constexpr int s = ks & 1;
    if constexpr (MODE != GM_W8) {
      static_for<NB>([&](auto nbc) {
        constexpr int nb = decltype(nbc)::value;
        static_for<TM>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          static_for<TN>([&](auto jc) {
            constexpr int j = (i & 1) ? TN - 1 - decltype(jc)::value : decltype(jc)::value;
            acc[nb][i][j] = mfma32<MODE>(fb[s][nb][j], fa[s][i], acc[nb][i][j]);
          });
        });
      });
      return;
    }
    static_for<NB>([&](auto nbc) {
      constexpr int nb = decltype(nbc)::value;
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        v4i bj;
        if constexpr (MODE != GM_W8) {
          bj = fb[s][nb][j];
        } else {
          constexpr int jp = ks >> 1, h = ks & 1;
          bj = __builtin_bit_cast(
              v4i, i8x8_to_v8h((uint32_t)fb[jp][nb][j][2 * h], (uint32_t)fb[jp][nb][j][2 * h + 1]));
        }
        static_for<TM>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
          if constexpr (MODE == GM_W8) acc[nb][i][j] = mfma32_f16(bj, fa[s][i], acc[nb][i][j]);
          else acc[nb][i][j] = mfma32<MODE>(bj, fa[s][i], acc[nb][i][j]);
        });
      });
    });
  };

  // One stage: the reads of step ks+1 are issued before the MFMAs of step
  // ks.  Before the last step's MFMAs the workgroup meets at the barrier
  // (every wave's loads of the next stage have landed, every wave is done
  // reading this one), the loads of stage kt+STAGES go into this stage's
  // buffer (DMA: 0 none, 1 a middle stage, 2 possibly the last stage) and
  // step 0 of the next stage is read, so the MFMA pipe never waits on a
  // barrier with an empty queue.  LAST: no next stage.  WAITN: direct loads
  // (per wave) that may still be in flight at the barrier -- those of the
  // stages after the next one.
  auto stage_body = [&](char* cur, char* nxt, int kt, auto dmac, auto lastc, auto waitc) __attribute__((always_inline)) {
    constexpr int DMA = decltype(dmac)::value;
    constexpr bool LAST = decltype(lastc)::value;
    constexpr int WAITN = decltype(waitc)::value;
    static_for<KSTEPS>([&](auto ksc) {
      constexpr int ks = decltype(ksc)::value;
      if constexpr (ks == KSTEPS - 1 && !LAST && DMA != 0) {
        // After the barrier: the next stage's first fragment reads, then the
        // direct loads of stage kt+2 alternating with this step's MFMAs, so
        // the MFMA pipe keeps running while the loads are issued (issued as
        // one burst, they stall the wave on the memory queue with its MFMAs
        // stuck behind them).
        wait_vm<WAITN>();
        lds_barrier();
        read_frags(nxt, std::integral_constant<int, 0>{});
        if constexpr (DMA == 1) dma_stage(cur, kt + STAGES, std::false_type{});
        if constexpr (DMA == 2) dma_stage(cur, kt + STAGES, std::true_type{});
        mfmas(ksc);
        interleave_reads_mfma_vmem<TM + NB * TN, NB * TN * TM, P>();
        __builtin_amdgcn_sched_barrier(0);
      } else {
        if constexpr (ks < KSTEPS - 1) {
          // the next step's reads spread between this step's MFMAs
          read_frags(cur, std::integral_constant<int, ks + 1>{});
          mfmas(ksc);
          interleave_reads_mfma_vmem<TM + NB * TN, NB * TN * TM, 0>();
          __builtin_amdgcn_sched_barrier(0);
        } else {
          if constexpr (!LAST) {
            wait_vm<WAITN>();
            lds_barrier();
            read_frags(nxt, std::integral_constant<int, 0>{});
          }
          __builtin_amdgcn_sched_barrier(0);
          mfmas(ksc);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    });
  };
  typedef std::integral_constant<int, 0> NoDma;
  typedef std::integral_constant<int, 2> LastDma;

  // Stage buffers (two stages): stage kt lives in st0 when kt - (nk & 1) is
  // even, so the final two stages are always (st0, st1) and the steady loop
  // needs no remainder; with an odd stage count stage 0 goes to st1 and is
  // peeled.  A single stage of K runs as three, the later two reading as
  // zeros (their loads are masked like any K tail).
  // The tile's scales go straight to LDS ahead of the first stage (wave 0:
  // row scales, 1: column scales, 2: second column scales): issued first,
  // they are covered by the prologue's wait for stage 0.  A null scale
  // pointer gives an empty buffer range, so its slot reads as zeros.
  float* scl = scl_all;  // the scale set of the tile being computed
  auto dma_scales = [&](float* dst) __attribute__((always_inline)) {
    static_assert(NW >= 2 + NB - 1, "one wave per scale vector");
    auto sc_rsrc = [](const float* ptr, int64_t first, int64_t n) {
      return __builtin_amdgcn_make_buffer_rsrc((void*)(ptr ? ptr + first : nullptr), 0,
                                               ptr ? (int)((n - first) * 4) : 0, 0x00020000);
    };
    if (wave == 0)
      dma16(sc_rsrc(MODE == GM_I8 ? p.row_scale : nullptr, m0, p.M), (char*)dst, lane * 16u, 0u);
    if (wave == 1) dma16(sc_rsrc(p.col_scale, n0, p.N), (char*)(dst + SC_ROWS), lane * 16u, 0u);
    if constexpr (NB == 2)
      if (wave == 2) dma16(sc_rsrc(p.col_scale2, n0, p.N), (char*)(dst + 2 * SC_ROWS), lane * 16u, 0u);
  };
  typedef std::integral_constant<int, 0> Wait0;
  typedef std::integral_constant<int, P> Wait1;  // one later stage's loads may be in flight
  typedef std::false_type More;
  auto first = [&](char* st) { read_frags(st, std::integral_constant<int, 0>{}); };
  // The direct loads of the first STAGES stages of the current tile.
  auto dma_prologue = [&]() __attribute__((always_inline)) {
    if constexpr (STAGES == 2) {
      if (nk & 1) {
        dma_stage(st1, 0, std::true_type{});
        dma_stage(st0, 1, std::true_type{});
      } else {
        dma_stage(st0, 0, std::true_type{});
        dma_stage(st1, 1, std::true_type{});
      }
    } else {
      // Three-stage ring.  Stage kt lives in buffer (kt + 3 - nk3 % 3) % 3,
      // so the final three stages are always (st0, st1, st2); the first
      // nk3 % 3 stages are peeled.  Fewer than three stages of K run as
      // three, the stages past K reading as zeros.
      const int r = (nk < 3 ? 3 : nk) % 3;
      if (r == 0) {
        dma_stage(st0, 0, std::true_type{});
        dma_stage(st1, 1, std::true_type{});
        dma_stage(st2, 2, std::true_type{});
      } else if (r == 1) {
        dma_stage(st2, 0, std::true_type{});
        dma_stage(st0, 1, std::true_type{});
        dma_stage(st1, 2, std::true_type{});
      } else {
        dma_stage(st1, 0, std::true_type{});
        dma_stage(st2, 1, std::true_type{});
        dma_stage(st0, 2, std::true_type{});
      }
    }
  };
  // The K loop over the prologue's stages and the rest.  EXTRA: memory
  // operations this wave issued after the prologue's loads (a persistent
  // workgroup's previous epilogue stores) that may still be in flight when
  // stage 0 is waited for -- vmcnt retires in issue order.
  auto k_loop = [&](auto extrac) __attribute__((always_inline)) {
    constexpr int EXTRA = decltype(extrac)::value;
    if constexpr (STAGES == 2) {
      const bool odd = nk & 1;
      wait_vm<P + EXTRA>();
      lds_barrier();
      int kt = 0;
      if (odd) {
        first(st1);
        stage_body(st1, st0, 0, LastDma{}, More{}, Wait0{});
        kt = 1;
      } else {
        first(st0);
      }
      // Steady state: straight-line pairs of stages (no conditional code, so
      // the accumulators keep one register class across iterations).
      for (; nk - kt > 2; kt += 2) {
        stage_body(st0, st1, kt, LastDma{}, More{}, Wait0{});
        stage_body(st1, st0, kt + 1, LastDma{}, More{}, Wait0{});
      }
      stage_body(st0, st1, kt, NoDma{}, More{}, Wait0{});
      stage_body(st1, st0, kt + 1, NoDma{}, std::true_type{}, Wait0{});
    } else {
      const int nk3 = nk < 3 ? 3 : nk;
      const int r = nk3 % 3;
      wait_vm<2 * P + EXTRA>();
      lds_barrier();
      int kt = 0;
      if (r == 1) {
        first(st2);
        stage_body(st2, st0, 0, LastDma{}, More{}, Wait1{});
        kt = 1;
      } else if (r == 2) {
        first(st1);
        stage_body(st1, st2, 0, LastDma{}, More{}, Wait1{});
        stage_body(st2, st0, 1, LastDma{}, More{}, Wait1{});
        kt = 2;
      } else {
        first(st0);
      }
      for (; nk3 - kt > 3; kt += 3) {
        stage_body(st0, st1, kt, LastDma{}, More{}, Wait1{});
        stage_body(st1, st2, kt + 1, LastDma{}, More{}, Wait1{});
        stage_body(st2, st0, kt + 2, LastDma{}, More{}, Wait1{});
      }
      stage_body(st0, st1, kt, NoDma{}, More{}, Wait1{});
      stage_body(st1, st2, kt + 1, NoDma{}, More{}, Wait0{});
      stage_body(st2, st0, kt + 2, NoDma{}, std::true_type{}, Wait0{});
    }
  };

  // K split merged in the kernel: every part stores its partial tile (in
  // register order: wave block, then (nb, i, j, g) 16-byte chunks of 64
  // lanes, so each store instruction writes one contiguous KiB) with the
  // agent-coherent policy, waits for the stores, and counts itself in on
  // the tile's counter; the part that counts last resets the counter, reads
  // every part's partial back (its own included) and adds them in part
  // order from zero -- the order of the separate merge kernel, so the
  // result is the same bit for bit -- then runs the epilogue.  The others
  // end here.  The protocol is the split decode GEMV's (hx_gemv.hip), with
  // the same gfx942 / gfx950 guarantees.  Returns false when this
  // workgroup ends.
  auto split_handoff = [&]() __attribute__((always_inline)) -> bool {
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__) && !defined(__gfx942__)
#error "in-kernel K-split merge: the last-arriver protocol is written for gfx942 / gfx950 (vmcnt counts stores)"
#endif
    constexpr int CH = NB * TM * TN * 4;  // 16-byte chunks per lane
    constexpr int TILE_BYTES = NB * BM * BN * 4;
    const int parts = gridDim.y;
    auto tile_rsrc = [&](int q) {
      char* base = reinterpret_cast<char*>(p.part) + ((int64_t)q * gridDim.x + blockIdx.x) * TILE_BYTES;
      return __builtin_amdgcn_make_buffer_rsrc((void*)base, 0, TILE_BYTES, 0x00020000);
    };
    // the lane's 16 bytes in the vector offset, the wave's chunk (uniform)
    // in the scalar offset
    const uint32_t voff = (uint32_t)lane * 16u;
    auto soff = [&](int c) -> uint32_t { return (uint32_t)((wave * CH + c) * 1024); };
    {
      const __amdgpu_buffer_rsrc_t mine = tile_rsrc(blockIdx.y);
      static_for<NB>([&](auto nbc) {
        static_for<TM>([&](auto ic) {
          static_for<TN>([&](auto jc) {
            static_for<4>([&](auto gc) {
              constexpr int nb = decltype(nbc)::value, i = decltype(ic)::value, j = decltype(jc)::value,
                            g = decltype(gc)::value;
              constexpr int c = ((nb * TM + i) * TN + j) * 4 + g;
              // the four components as one sub-vector, cast whole: hipcc
              // compiles a bit cast of a single vector component as a cast
              // of component 0
              const Acc& v = acc[nb][i][j];
              const v4i d = __builtin_bit_cast(v4i, __builtin_shufflevector(v, v, 4 * g, 4 * g + 1, 4 * g + 2,
                                                                            4 * g + 3));
              __builtin_amdgcn_raw_buffer_store_b128(d, mine, voff, soff(c), kAgentCoherent);
            });
          });
        });
      });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0)
      is_last_part = __hip_atomic_fetch_add(p.cnt + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                     (unsigned)(parts - 1);
    __syncthreads();
    if (!is_last_part) return false;
    if (tid == 0) __hip_atomic_store(p.cnt + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // one (nb, i, j) sub-tile at a time: its four chunks of every part
    static_for<NB>([&](auto nbc) {
      static_for<TM>([&](auto ic) {
        static_for<TN>([&](auto jc) {
          constexpr int nb = decltype(nbc)::value, i = decltype(ic)::value, j = decltype(jc)::value;
          constexpr int c0 = ((nb * TM + i) * TN + j) * 4;
          Acc& v = acc[nb][i][j];
          v = Acc{};
          for (int q = 0; q < parts; ++q) {
            const __amdgpu_buffer_rsrc_t r = tile_rsrc(q);
            typedef decltype(__builtin_shufflevector(v, v, 0, 1, 2, 3)) Part4;  // v4i or v4f
            Part4 d[4];
            static_for<4>([&](auto gc) {
              constexpr int g = decltype(gc)::value;
              d[g] = __builtin_bit_cast(Part4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff(c0 + g),
                                                                                     kAgentCoherent));
            });
            static_for<4>([&](auto gc) {
              constexpr int g = decltype(gc)::value;
              static_for<4>([&](auto ec) {
                constexpr int e = decltype(ec)::value;
                if constexpr (MODE == GM_I8)
                  v[4 * g + e] = (int)((uint32_t)v[4 * g + e] + (uint32_t)d[g][e]);
                else
                  v[4 * g + e] = v[4 * g + e] + d[g][e];
              });
            });
          }
          __builtin_amdgcn_sched_barrier(0);
        });
      });
    });
    return true;
  };

  // ---- epilogue ----------------------------------------------------------
  // Lane (lrow, lg) holds row wm*WTM + 32*i + lrow, columns
  // wn*WTN + 32*j + 8*g + 4*lg + (0..3) of the tile in registers 4g..4g+3 of
  // sub-tile (i, j).  Stored straight from that layout, every store
  // instruction would write 16 bytes into each of 32 rows (32 partial-line
  // requests).  Instead each wave converts its block to the output type in a
  // private LDS region (the stage buffers are free now), row-major with the
  // 16-byte chunk XOR-swizzled by row (conflict-free 8/16-byte writes and
  // 16-byte reads), and reads it back so that every lane stores 16
  // consecutive bytes and a wave store covers whole rows.
  //
  // The epilogue is straight-line code: the output type is a compile-time
  // variant chosen once, the scales come from LDS (fetched in the prologue;
  // an absent scale reads as 1.0, and multiplying by 1.0 is exact, so the
  // result equals skipping the multiply), and residual reads use clamped
  // in-bounds indices (values for rows/columns past the edge are never
  // stored).  A per-element test of the output type or of an optional
  // argument would put a branch, and a wait for every load behind it, on
  // each element.  The block goes out in passes of 32 rows, so the
  // conversion of one pass overlaps the stores of the previous one; all
  // loads of a pass (residual) are issued before any store of that pass, so
  // a residual that aliases C is read first.  The output stores are
  // non-temporal: the tile is written once and not read back, and streamed
  // stores drain to memory as they go instead of waiting in L2 for the
  // end-of-kernel write-back.
  int64_t row0w = 0, col0w = 0;   // the finished tile's wave block
  const float* scl_e = scl;        // and its scale set
  const bool has_rs = MODE == GM_I8 && p.row_scale != nullptr;
  const bool has_cs = p.col_scale != nullptr;
  const bool has_cs2 = NB == 2 && p.col_scale2 != nullptr;
  // scale of sub-tile row i / columns (j, g) of this lane, read from LDS
  // where it is used (holding a whole wave block's scales in registers
  // would cost 16 registers per sub-tile column)
  auto row_scale_of = [&](int i) -> float { return has_rs ? scl_e[wm * WTM + i * 32 + lrow] : 1.f; };
  auto col_scale_of = [&](int j, int g, int which) -> v4f {
    const bool has = which ? has_cs2 : has_cs;
    const int c = wn * WTN + j * 32 + 8 * g + 4 * lg;
    return has ? *reinterpret_cast<const v4f*>(scl_e + (1 + which) * SC_ROWS + c) : v4f{1.f, 1.f, 1.f, 1.f};
  };
  const bool has_res = MODE != GM_I8 && EPI != GE_SWIGLU && p.res != nullptr;

  // OK: output kind (DT_I32 / DT_F32 / DT_F16 / DT_BF16), a compile-time value
  auto epilogue = [&](auto okc) __attribute__((always_inline)) {
    constexpr int OK = decltype(okc)::value;
    constexpr int ES = (OK == DT_I32 || OK == DT_F32) ? 4 : 2;  // output element bytes
    constexpr int RB = WTN * ES;                 // bytes per row of the wave block
    constexpr int PER_ARRAY = (NW + 1) / 2;      // wave regions per stage buffer
    constexpr int REGION = STAGE / PER_ARRAY;
    constexpr int TMP = 1;  // 32-row passes
    static_assert(TMP >= 1 && TM % TMP == 0 && TMP * 32 * RB <= REGION, "epilogue region");
    static_assert(RB >= 64 && (1024 % RB == 0 || RB % 1024 == 0), "epilogue row bytes");
    auto swz_out = [](int row) -> int {
      if constexpr (RB == 64) return (row >> 2) & 3;
      else if constexpr (RB == 128) return (row >> 1) & 7;
      else return row & 15;
    };
    static_assert(!PERSIST || ES == 2, "persistent: 16-bit outputs");
    char* region = PERSIST ? stg + wave * STG_WAVE
                           : (wave < PER_ARRAY ? st0 : st1) + (wave % PER_ARRAY) * (TMP * 32 * RB);
    // the wave block's output rows: rows row0w.. (up to the matrix end),
    // columns from col0w; the fast path keeps 256 rows within 2^31 bytes
    const int64_t out_rows = p.M - row0w;
    const int64_t out_bytes = out_rows > 0 ? (out_rows - 1) * p.ldc * ES + (p.N - col0w) * ES : 0;
    const __amdgpu_buffer_rsrc_t rc_out = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<char*>(p.c) + (row0w * p.ldc + col0w) * ES, 0,
        (int)(out_bytes < 0x7fffffff ? out_bytes : 0x7fffffff), 0x00020000);
    static_for<TM / TMP>([&](auto pc) {
      constexpr int pp = decltype(pc)::value;
      // 1) this pass's sub-tile rows -> LDS, in the output type
      static_for<TN>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        // residual of sub-tile column j of this pass (float GE_STORE only)
        v4f res[TMP][4];
        if constexpr (MODE != GM_I8 && EPI != GE_SWIGLU) {
          static_for<TMP>([&](auto ic) {
            constexpr int ii = decltype(ic)::value;
            static_for<4>([&](auto gc) {
              constexpr int g = decltype(gc)::value;
              if (has_res) {
                const int64_t row = min(row0w + (pp * TMP + ii) * 32 + lrow, p.M - 1);
                const int64_t col = min(col0w + j * 32 + 8 * g + 4 * lg, p.N - 4);
                res[ii][g] = load4(p.res, p.res_dtype, row * p.ldr + col);
              } else {
                res[ii][g] = v4f{0.f, 0.f, 0.f, 0.f};
              }
            });
          });
        }
        v4f cs[4], cs2[4];
        static_for<4>([&](auto gc) {
          constexpr int g = decltype(gc)::value;
          cs[g] = col_scale_of(j, g, 0);
          if constexpr (NB == 2) cs2[g] = col_scale_of(j, g, 1);
        });
        static_for<TMP>([&](auto ic) {
          constexpr int ii = decltype(ic)::value;
          constexpr int i = pp * TMP + ii;
          const int rl = ii * 32 + lrow;
          const float rs = row_scale_of(i);
          static_for<4>([&](auto gc) {
            constexpr int g = decltype(gc)::value;
            const int byte = (j * 32 + 8 * g + 4 * lg) * ES;
            char* dst = region + rl * RB + (((byte >> 4) ^ swz_out(rl)) << 4) + (byte & 15);
            if constexpr (MODE == GM_I8 && OK == DT_I32) {
              *reinterpret_cast<v4i*>(dst) =
                  v4i{(int)acc[0][i][j][4 * g], (int)acc[0][i][j][4 * g + 1],
                      (int)acc[0][i][j][4 * g + 2], (int)acc[0][i][j][4 * g + 3]};
            } else {
              float v[4];
              static_for<4>([&](auto qc) {
                constexpr int q = decltype(qc)::value;
                if constexpr (MODE == GM_I8) {
                  v[q] = ((float)acc[0][i][j][4 * g + q] * rs) * cs[g][q];
                } else if constexpr (EPI == GE_SWIGLU) {
                  const float gt =
                      f16_bits_to_f32(f32_to_f16_bits(acc[0][i][j][4 * g + q] * cs[g][q]));
                  const float up =
                      f16_bits_to_f32(f32_to_f16_bits(acc[NB - 1][i][j][4 * g + q] * cs2[g][q]));
                  const float sg = gt / (1.0f + fast_exp(-gt));
                  v[q] = sg * up;
                } else {
                  const float t = acc[0][i][j][4 * g + q] * cs[g][q];
                  v[q] = has_res ? t + res[ii][g][q] : t;
                }
              });
              if constexpr (ES == 4) {
                *reinterpret_cast<v4f*>(dst) = v4f{v[0], v[1], v[2], v[3]};
              } else if constexpr (OK == DT_BF16) {
                const uint32_t lo = (uint32_t)f32_to_bf16(v[0]) | ((uint32_t)f32_to_bf16(v[1]) << 16);
                const uint32_t hi = (uint32_t)f32_to_bf16(v[2]) | ((uint32_t)f32_to_bf16(v[3]) << 16);
                *reinterpret_cast<v2i*>(dst) = v2i{(int)lo, (int)hi};
              } else {
                *reinterpret_cast<v2i*>(dst) =
                    v2i{(int)f32x2_to_f16x2(v[0], v[1]), (int)f32x2_to_f16x2(v[2], v[3])};
              }
            }
          });
        });
      });
      // 2) LDS -> global: 16 bytes per lane, whole rows per wave store.
      // Full chunks go out as buffer stores with system-scope coherence
      // (write-through): the tile streams to memory as it is written instead
      // of sitting dirty in L2 for the end-of-kernel write-back, which with
      // every CU storing at once left the chip idle for several us (6 us of
      // 67 at 4096^3 int8 against non-temporal flat stores).  The wave's
      // block is the descriptor base, so offsets stay within 32 bits.
      constexpr int NI = TMP * 32 * RB / 1024;
      constexpr int EPC = 16 / ES;  // elements per 16-byte chunk
      static_for<NI>([&](auto qc) {
        constexpr int q = decltype(qc)::value;
        const int byte = q * 1024 + lane * 16;
        const int rl = byte / RB, c = (byte % RB) >> 4;
        const v4i d = *reinterpret_cast<const v4i*>(region + rl * RB + ((c ^ swz_out(rl)) << 4));
        const int64_t row = row0w + pp * TMP * 32 + rl;
        const int64_t col = col0w + c * EPC;
        const uint32_t off = (uint32_t)((((int64_t)(pp * TMP * 32 + rl)) * p.ldc + c * EPC) * ES);
        if constexpr (!EDGE) {
          // interior tiles: every row and chunk is in range, so every wave
          // issues exactly TM * NI stores (a persistent workgroup's next
          // stage wait counts on it)
          __builtin_amdgcn_raw_buffer_store_b128(d, rc_out, off, 0, kStoreWriteThrough);
        } else if (row < p.M) {
          if (col + EPC <= p.N) {
            __builtin_amdgcn_raw_buffer_store_b128(d, rc_out, off, 0, kStoreWriteThrough);
          } else if (ES == 2 && col < p.N) {
            char* out = reinterpret_cast<char*>(p.c) + (row * p.ldc + col) * ES;
            *reinterpret_cast<v2i*>(out) = v2i{d[0], d[1]};
          }
        }
      });
    });
  };
  // the epilogue of the tile whose wave block starts at (row0w, col0w)
  auto epilogue_any = [&]() __attribute__((always_inline)) {
    if constexpr (PERSIST) {
      // launch_one runs persistent configs for 16-bit outputs only
      if (p.out_dtype == DT_BF16) epilogue(std::integral_constant<int, DT_BF16>{});
      else epilogue(std::integral_constant<int, DT_F16>{});
    } else {
      switch (p.out_dtype) {
        case DT_I32: if constexpr (MODE == GM_I8) epilogue(std::integral_constant<int, DT_I32>{}); break;
        case DT_F32: if constexpr (EPI != GE_SWIGLU) epilogue(std::integral_constant<int, DT_F32>{}); break;
        case DT_BF16: epilogue(std::integral_constant<int, DT_BF16>{}); break;
        default: epilogue(std::integral_constant<int, DT_F16>{}); break;
      }
    }
  };
  auto zero_acc = [&]() __attribute__((always_inline)) {
    static_for<NB>([&](auto nbc) {
      static_for<TM>([&](auto ic) {
        static_for<TN>([&](auto jc) {
          acc[decltype(nbc)::value][decltype(ic)::value][decltype(jc)::value] = Acc{};
        });
      });
    });
  };
  (void)zero_acc;

  if constexpr (!PERSIST) {
    dma_scales(scl);
    dma_prologue();
    k_loop(std::integral_constant<int, 0>{});
    if constexpr (SPLITM) {
      if (!split_handoff()) {
        clock_out();
        return;
      }
    }
    lds_barrier();  // every wave is done reading the stage buffers
    row0w = m0 + wm * WTM;
    col0w = n0 + wn * WTN;
    scl_e = scl;
    epilogue_any();
  } else {
    // stores per wave in one epilogue (16-bit output, interior tiles)
    constexpr int NS = TM * (32 * WTN * 2 / 1024);
    static_assert(STAGES * P + NS < 64, "vmcnt range");
    dma_scales(scl);
    dma_prologue();
    bool first_tile = true;
    for (;;) {
      if (first_tile) k_loop(std::integral_constant<int, 0>{});
      else k_loop(std::integral_constant<int, NS>{});
      lds_barrier();  // every wave is done reading the stage buffers
      row0w = m0 + wm * WTM;
      col0w = n0 + wn * WTN;
      scl_e = scl;
      // the next tile's scales and first stages go out before this tile's
      // epilogue, so they load while it converts and stores
      const bool more = ++t_cur < t_end;
      if (more) {
        int tm_, tn_;
        tile_of_lin(t_cur, tiles_m, tiles_n, tm_, tn_);
        set_tile(tm_, tn_);
        scl = scl == scl_all ? scl_all + (1 + NB) * SC_ROWS : scl_all;
        dma_scales(scl);
        dma_prologue();
      }
      epilogue_any();
      if (!more) break;
      first_tile = false;
      zero_acc();
      // what derives from lane and wave is recomputed for the next tile
      // rather than held across its K loop
      int t = tid;
      asm volatile("" : "+v"(t));
      lane = t & 63;
      wave = __builtin_amdgcn_readfirstlane(t >> 6);
      lrow = lane & 31;
      lg = lane >> 5;
      wm = wave / WN;
      wn = wave % WN;
    }
  }
  clock_out();
}


// ---------------------------------------------------------------------------
// Config table.  The autotuner searches over these instantiations.
// ---------------------------------------------------------------------------
typedef void (*GemmLaunch)(const GemmArgs&, hipStream_t);

// PERSIST configs run the persistent kernel on interior shapes with 16-bit
// outputs and no K split (one workgroup per CU, or fewer when there are
// fewer tiles), and the one-tile-per-workgroup kernel of the same tile
// otherwise.
// SPLITM configs (the K-split ones) merge their parts inside the kernel
// when the launch brings per-tile counters, and through launch_gemm's
// merge kernel otherwise.
template <int MODE, int BM, int BN, int WM, int WN, int EPI, int SB = 128, int STAGES = 2, int MINW = 1,
          bool PERSIST = false, bool SPLITM = false>
static void launch_one(const GemmArgs& a, hipStream_t s) {
  const int64_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  const unsigned parts = a.k_split > 0 ? (unsigned)((a.K + a.k_split - 1) / a.k_split) : 1u;
  const dim3 grid((unsigned)tiles, parts), block(64 * WM * WN);
  const bool edge = a.M % BM != 0 || a.N % BN != 0;
  if constexpr (PERSIST) {
    if (!edge && !a.b_kn && parts == 1 && (a.out_dtype == DT_F16 || a.out_dtype == DT_BF16)) {
      const int64_t g = tiles < gemm_num_cus() ? tiles : gemm_num_cus();
      gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, false, false, STAGES, true>
          <<<dim3((unsigned)g), block, 0, s>>>(a);
      return;
    }
  }
  if constexpr (SPLITM && EPI == GE_STORE) {
    if (parts > 1 && a.cnt) {
      if constexpr (MODE == GM_F16 || MODE == GM_BF16 || MODE == GM_I8) {
        if (a.b_kn) {
          if (edge) gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, true, true, STAGES, false, true><<<grid, block, 0, s>>>(a);
          else gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, false, true, STAGES, false, true><<<grid, block, 0, s>>>(a);
          return;
        }
      }
      if (edge) gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, true, false, STAGES, false, true><<<grid, block, 0, s>>>(a);
      else gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, false, false, STAGES, false, true><<<grid, block, 0, s>>>(a);
      return;
    }
  }
  if constexpr ((MODE == GM_F16 || MODE == GM_BF16 || MODE == GM_I8) && EPI == GE_STORE) {
    if (a.b_kn) {
      if (edge) gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, true, true, STAGES><<<grid, block, 0, s>>>(a);
      else gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, false, true, STAGES><<<grid, block, 0, s>>>(a);
      return;
    }
  }
  if (edge) gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, true, false, STAGES><<<grid, block, 0, s>>>(a);
  else gemm_kernel<MODE, BM, BN, WM, WN, EPI, SB, MINW, false, false, STAGES><<<grid, block, 0, s>>>(a);
}

struct GemmEntry {
  GemmConfig cfg;
  GemmLaunch fn;
};

// occ = workgroups a CU holds at once, rate = relative output throughput of
// one CU at that occupancy, both measured on MI355X at 4096^3 (int8, fp16)
// and 2048x11008x4096 (W8A16); they drive the untuned default choice.
#define HX_GEMM_CFGS(MODE)                                                                         \
  {{256, 256, 2, 2, GE_STORE, "256x256_w2x2", 1, 0.74f}, &launch_one<MODE, 256, 256, 2, 2, GE_STORE>}, \
  {{256, 128, 2, 2, GE_STORE, "256x128_w2x2", 1, 0.77f}, &launch_one<MODE, 256, 128, 2, 2, GE_STORE>}, \
  {{128, 256, 2, 2, GE_STORE, "128x256_w2x2", 1, 0.77f}, &launch_one<MODE, 128, 256, 2, 2, GE_STORE>}, \
  {{128, 128, 2, 2, GE_STORE, "128x128_w2x2", 2, 0.89f}, &launch_one<MODE, 128, 128, 2, 2, GE_STORE>}, \
  {{256, 256, 2, 4, GE_STORE, "256x256_w2x4", 1, 1.00f}, &launch_one<MODE, 256, 256, 2, 4, GE_STORE>}, \
  {{64, 64, 2, 2, GE_STORE, "64x64_w2x2", 4, 0.61f}, &launch_one<MODE, 64, 64, 2, 2, GE_STORE>}


// One table per operand mode, each in its own translation unit
// (hx_gemm_{i8,f16,bf16,w8}.hip) so that the instantiations compile in
// parallel.
const GemmEntry* gemm_table_i8(int& n);
const GemmEntry* gemm_table_f16(int& n);
const GemmEntry* gemm_table_bf16(int& n);
const GemmEntry* gemm_table_w8(int& n);

}  // namespace hx
