// hx_internal.hpp -- host-side declarations shared by the kernel translation
// units and the C ABI layer (hx_api.cpp).  Nothing here is exported.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hx {

enum : int {
  HXI_OK = 0,
  HXI_ERR_ARG = -1,
  HXI_ERR_SHAPE = -2,
  HXI_ERR_DTYPE = -3,
  HXI_ERR_LAYOUT = -4,
  HXI_ERR_HIP = -5,
  HXI_ERR_NOMEM = -6,
  HXI_ERR_UNSUPPORTED = -7,
  HXI_ERR_CAPTURE = -8,  // set-up refused under graph capture (message recorded)
};

// ---- row kernels (hx_rows.hip) -------------------------------------------
// cfg: an index into the row configurations (row_config_*), -1 for the
// untuned default of the shape.
int launch_softmax(int dtype, const void* x, int64_t ldx, void* y, int64_t ldy,
                   int64_t rows, int64_t cols, hipStream_t s, int cfg = -1);
int launch_rmsnorm(int dtype, const void* x, int64_t ldx, const void* gamma, float eps,
                   void* y, int64_t ldy, int64_t rows, int64_t cols, hipStream_t s, int cfg = -1);
int launch_layernorm(int dtype, const void* x, int64_t ldx, const void* w, const void* b,
                     float eps, void* y, int64_t ldy, float* mean, float* rstd,
                     int64_t rows, int64_t cols, hipStream_t s, int cfg = -1);
int launch_silu_mul_f16(const void* g, int64_t ldg, const void* u, int64_t ldu, void* o,
                        int64_t ldo, int64_t rows, int64_t cols, hipStream_t s);
// Rows longer than the launches above hold in registers (they return
// HXI_ERR_UNSUPPORTED without launching): two streaming passes, with
// row_long_ws_bytes() of per-segment statistics in `ws`.
enum RowOpCode : int { ROW_OP_SOFTMAX = 0, ROW_OP_RMSNORM = 1, ROW_OP_LAYERNORM = 2 };
// Row configurations: index 0 runs one row per workgroup; the others run the
// streaming form with row_config_per_cu() workgroups per CU.
int row_config_count();
const char* row_config_name(int cfg);
int row_config_per_cu(int cfg);
// Untuned choice (op: RowOpCode, dtype: HX_* code).
int row_default_config(int op, int dtype, int64_t rows, int64_t cols);
size_t row_long_ws_bytes(int dtype, int64_t rows, int64_t cols);
int launch_row_long(int op, int dtype, const void* x, int64_t ldx, const void* w, const void* b, float eps,
                    void* y, int64_t ldy, float* mean, float* rstd, int64_t rows, int64_t cols, void* ws,
                    hipStream_t s);

// ---- MFMA GEMM (hx_gemm.hip) ---------------------------------------------
// Operand modes.  B is always consumed K-contiguous ([N][K], "NK").
enum GemmMode : int {
  GM_I8 = 0,    // int8 x int8 -> int32      (v_mfma_i32_32x32x32_i8)
  GM_F16 = 1,   // f16 x f16 -> f32          (v_mfma_f32_32x32x16_f16)
  GM_BF16 = 2,  // bf16 x bf16 -> f32        (v_mfma_f32_32x32x16_bf16)
  GM_W8 = 3,    // f16 x int8 -> f32, int8 widened to f16 in registers
  GM_COUNT = 4,
};

enum GemmEpi : int { GE_STORE = 0, GE_SWIGLU = 1 };

struct GemmArgs {
  const void* a; int64_t lda;   // [M][K], elements
  const void* b; int64_t ldb;   // [N][K], elements ([K][N] when b_kn)
  const void* b2;               // second weight for GE_SWIGLU (same ldb)
  void* c; int64_t ldc;         // [M][N]
  int64_t M, N, K;
  int out_dtype;                // DT_I32 / DT_F16 / DT_BF16 / DT_F32
  const float* row_scale;       // [M] (int8 dequant), may be null
  const float* col_scale;       // [N], may be null
  const float* col_scale2;      // [N] scale of b2 (GE_SWIGLU)
  const void* res; int64_t ldr; int res_dtype;  // residual, may be null
  int b_kn;                     // f16 / bf16 only: b is [K][N] (N contiguous)
  // K split: the kernel runs gridDim.y parts of k_split elements, each
  // writing binary32 (int8: int32) partials to its [M][N] slice of c;
  // `part` is the partial buffer launch_gemm uses for a split config
  int64_t k_split;
  float* part;
  // K split merged inside the kernel (null: a second kernel merges): one
  // counter per output tile, zero on entry and returned to zero; the
  // partials are then [parts][tiles][BM*BN] in the kernel's register order
  unsigned* cnt;
  // measurement hook (null: off): every workgroup adds its elapsed
  // shader-clock cycles, constant-rate ticks and 1 to clk[0..2]
  unsigned long long* clk;
};

struct GemmConfig {
  int bm, bn, wm, wn;   // block tile and wave grid
  int epi;              // GemmEpi
  const char* name;
  int occ;              // workgroups resident per CU (LDS / register limit)
  float rate;           // measured output throughput of one CU, relative
  int ksplit = 0;       // K parts (0 or 1: none); partials merged by the last part of each tile
  int sb = 128;         // bytes of A per row in one K stage (64, 128, 256)
  int stages = 2;       // K stages resident in LDS at once (2 or 3)
  int persist = 0;      // 1: one workgroup per CU walks consecutive M-tiles of a B strip
};
// Partial-buffer bytes a launch of config cfg_idx needs (0 without a K split).
size_t gemm_part_bytes(int mode, int cfg_idx, const GemmArgs& a);
// Output tiles of a launch of config cfg_idx (the counters an in-kernel
// K-split merge uses).
int64_t gemm_tiles(int mode, int cfg_idx, const GemmArgs& a);
// The clock hook: the per-device counters launch_gemm passes to the tiled
// kernels while it is on (null: off).
void gemm_clock_target(int dev, unsigned long long* clk);

int gemm_config_count(int mode);
// Compute units of the current device (the persistent configs' grid).
int gemm_num_cus();
const GemmConfig* gemm_config(int mode, int idx);
// Default (untuned) config index for a shape.
int gemm_default_config(int mode, int epi, int64_t M, int64_t N, int64_t K);
// True when the fast kernel's alignment preconditions hold for these args;
// otherwise gemm_fast_refusal names the first one that fails.
bool gemm_fast_ok(int mode, const GemmArgs& a);
const char* gemm_fast_refusal(int mode, const GemmArgs& a);
int launch_gemm(int mode, int cfg_idx, const GemmArgs& a, hipStream_t s);
// Any shape / alignment; simple tiled kernel, same arithmetic contract.
int launch_gemm_generic(int mode, const GemmArgs& a, hipStream_t s);

// ---- decode GEMM / GEMV, M <= 16 (hx_gemv.hip) ---------------------------
struct GemvArgs {
  const void* x; int64_t ldx;   // f16 [M][K] (bf16 with bf16 weights)
  const int8_t* w; int64_t ldw; // int8 [N][K] (unregistered int8 weights)
  const float* scale;           // [N], may be null (scale 1)
  const uint16_t* scale16;      // [N] f16 scale, used when `scale` is null
  void* y; int64_t ldy;         // [M][N], the activations' type
  int64_t M, N, K;
  // optional SwiGLU gate [M][N] f16 (streaming kernel, f16 output): each
  // output becomes RNE(silu(gate) * RNE(result))
  const uint16_t* gate = nullptr; int64_t ldg = 0;
  // K split over workgroups (set by the launcher from the config): `parts`
  // workgroups per column-tile group each reduce a contiguous K range into
  // binary32 partials [parts][M][N]; the last of them to finish (one
  // counter per group, returned to zero by that workgroup) adds the parts
  // in part order and finishes the outputs.  Null buffers: the launcher
  // takes the stream's own.
  int parts = 1;
  float* part = nullptr;
  unsigned* cnt = nullptr;
};
struct GemvConfig {
  int ct, kw;        // 16-column tiles per workgroup, waves splitting K
  const char* name;
  int xl;            // activations staged in LDS (M <= 4, rows within 64 KiB)
  int base;          // config that runs outside the xl or split limits
  int mb;            // 16-row activation blocks (M <= 16 mb)
  int split = 1;     // workgroups per column-tile group (K parts), M > 4 only
};
// Counters the split GEMV may use per launch (one per column-tile group).
constexpr int64_t kGemvSplitCounters = 16384;
// Partial bytes a launch of config `cfg` needs at this shape (0: it does
// not split here).
size_t gemv_split_bytes(int cfg, int64_t M, int64_t N);
// Whether config `cfg` splits K at M rows and N columns.
bool gemv_split_takes(const GemvConfig& c, int64_t M, int64_t N);
// The stream's split buffers (at least part_bytes of partials and
// kGemvSplitCounters zeroed counters); defined by the API layer.
int gemv_split_buffers(hipStream_t s, size_t part_bytes, float** part, unsigned** cnt);
// Largest M the decode GEMV takes (row-block configs).
constexpr int kGemvMaxRows = 64;
// Where 16 < M <= kGemvRowsMaxM rows take the decode GEMV's row blocks
// rather than the tiled GEMM: on a registered int8 weight's packed image
// always; on an f16 / bf16 packed image when N >= kGemvRowsMinN (fewer
// 16-column tiles leave most CUs idle); on a [N][K] weight read in place
// (sixteen 64-byte runs per wave load, not one contiguous KiB) when also
// N <= kGemvRowsInPlaceMaxN.  The kernels themselves take kGemvMaxRows.
constexpr int64_t kGemvRowsMaxM = 32;
constexpr int64_t kGemvRowsMinN = 2048;
constexpr int64_t kGemvRowsInPlaceMaxN = 4096;
// A registered int8 weight's packed image also takes four row blocks
// (32 < M <= 64) where they beat the tiled GEMM (interleaved A/B, rotating
// images): the down projection's shapes (129..256 tiles of 16 columns,
// K >= 8192) up to 64 rows, three tiles per CU (641..768 tiles, N = 11008)
// up to 48 rows (at 64 rows the tiled GEMM is 3% faster there).  In the FFN
// block (ffn) the gate and up projections take them up to 64 rows: two
// GEMVs then beat the fused gate/up GEMM.
constexpr int64_t kGemvRowsMaxMI8 = 64;
inline bool gemv_rows4_i8(int64_t M, int64_t N, int64_t K, bool ffn = false) {
  const int64_t tiles = (N + 15) / 16;
  if (M <= kGemvRowsMaxM || M > kGemvRowsMaxMI8) return false;
  if (tiles > 128 && tiles <= 256 && K >= 8192) return true;
  return (tiles + 255) / 256 == 3 && (ffn || M <= 48);
}
// An f16 / bf16 packed image takes them (32 < M <= 64) at three tiles per
// CU with K >= 4096 (N = 11008, K = 4096, M = 33 / 48 / 64: 21.97 / 24.54 /
// 28.01 us against 33.25 / 34.73 / 34.11 tiled); on the down projection's
// shape (4096 x 11008) the tiled GEMM stays ahead (28.0-28.6 against
// 29.4-34.2 us).
inline bool gemv_rows4_f16(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles = (N + 15) / 16;
  return M > kGemvRowsMaxM && M <= kGemvRowsMaxMI8 && (tiles + 255) / 256 == 3 && K >= 4096;
}
inline bool gemv_rows_route(int64_t M, int64_t N, bool packed, bool int8 = false, int64_t K = 0) {
  if (M <= 16) return true;
  if (packed && int8 && gemv_rows4_i8(M, N, K)) return true;
  if (packed && !int8 && gemv_rows4_f16(M, N, K)) return true;
  if (M > kGemvRowsMaxM) return false;
  if (packed && int8) return true;
  if (N < kGemvRowsMinN) return false;
  return packed || N <= kGemvRowsInPlaceMaxN;
}
// Untuned row-block config for 16 < M <= kGemvMaxRows.
int gemv_rows_default(int64_t M, int64_t N, int64_t K);
// Whether config c may stage M activation rows of K (wt: the weight's type)
// in LDS; a config that may not runs as its base config.
bool gemv_xl_fits(const GemvConfig& c, int64_t M, int64_t K, int wt);
bool gemv_fast_ok(const GemvArgs& a);
const char* gemv_fast_refusal(const GemvArgs& a);
// Column tiles per workgroup (1, 2 or 4 as index 0..2) of the [N][K] kernel.
int gemv_raw_config(const GemvArgs& a);
// [N][K] weight GEMV (unregistered weights).
int launch_gemv_w8a16(const GemvArgs& a, hipStream_t s);
// Fragment-packed resident image for the decode GEMV (see hx_gemv.hip).
int64_t gemv_packed_bytes(int64_t N, int64_t K);
int launch_gemv_pack(const int8_t* w_nk, int64_t ldw, int64_t N, int64_t K, int8_t* out, hipStream_t s);
int gemv_packed_config_count();
const GemvConfig* gemv_packed_config(int idx);
int launch_gemv_packed(int cfg_idx, const GemvArgs& a, const int8_t* packed, hipStream_t s);
// f16 / bf16 weights: the 16-bit fragment-packed image (16 columns x 32 k per
// KiB block) of a registered weight, and the decode GEMV over it.
int64_t gemv_packed16_bytes(int64_t N, int64_t K);
int launch_gemv_pack16(const uint16_t* w_nk, int64_t ldw, int64_t N, int64_t K, uint16_t* out, hipStream_t s);
int launch_gemv_packed16(int cfg_idx, int wt, const GemvArgs& a, const void* packed, hipStream_t s);
// One activation row (M = 1) against a K-contiguous [N][K] matrix read in
// place, whole rows per wave in contiguous KiBs; K <= 8192.  Null when the
// shape is taken.
const char* rowdot_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw);
int launch_rowdot(int wt, const GemvArgs& a, const void* w, int64_t ldw, hipStream_t s);
// Weights read in place from a K-contiguous [N][K] matrix with row stride
// ldw (elements): f16 / bf16 (wt = DT_F16 / DT_BF16), or int8 (DT_I8, f16
// activations); the same config table as the packed int8 kernel.  Null when
// the shape and layout are taken, else the refusal.
const char* gemv_hw_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw);
int launch_gemv_hw(int cfg_idx, int wt, const GemvArgs& a, const void* w, int64_t ldw, hipStream_t s);
// Weights in the [K][N] orientation (row stride ldw), read in place: f16 /
// bf16, or int8 (wt = DT_I8) with f16 activations.  K is split over `parts`
// workgroups per column block, whose binary32 partials (gemv_kn_part_bytes)
// are summed by a second kernel when > 1.
const char* gemv_kn_refusal(int wt, const GemvArgs& a, const void* w, int64_t ldw);
int gemv_kn_parts(int wt, const GemvArgs& a);
size_t gemv_kn_part_bytes(const GemvArgs& a, int parts);
int launch_gemv_kn(int wt, const GemvArgs& a, const void* w, int64_t ldw, int parts, float* part, hipStream_t s);

// ---- scaled-dot-product attention (hx_attn.hip) --------------------------
struct AttnArgs {
  const void* q; const void* k; const void* v; void* o;  // [Z][H][N][D], D contiguous
  int64_t sq[3], sk[3], sv[3], so[3];                     // element strides of Z, H, N
  int64_t Z, H, Nq, Nk, D;
  float scale;
  int64_t causal_offset;  // causal: key <= query + offset is visible
  int splits;             // key-range splits per (head, query block); 1 = single pass
  float* part;            // split partials (attn_part_bytes), used when splits > 1
};
// Null when the fused kernel takes these args, else the first refusal.
const char* attn_refusal(const AttnArgs& a);
// Key-range splits for a launch of these args (1 when the heads and query
// blocks alone occupy the chip), and the partial-result bytes they need.
int attn_splits(const AttnArgs& a);
size_t attn_part_bytes(const AttnArgs& a);
int launch_attention(int dtype, bool causal, const AttnArgs& a, hipStream_t s);

// ---- layout utilities (hx_pack.hip) --------------------------------------
// dst[c][r] = src[r][c] for a rows x cols matrix of 1/2/4-byte elements.
int launch_transpose(const void* src, int64_t lds, void* dst, int64_t ldd, int64_t rows,
                     int64_t cols, int elem_bytes, hipStream_t s);
// f32 [rows][cols] (row stride lds) -> dense f16, (x + 0) rounded to
// nearest even (-0 becomes +0): the reference's f32 pack quantisation.
// n 32-bit words of p set to v by a kernel (graph-capturable, unlike a
// memset node).
int launch_fill_u32(unsigned* p, int64_t n, unsigned v, hipStream_t s);
int launch_f32_to_f16_rne(const float* src, int64_t lds, uint16_t* dst, int64_t rows, int64_t cols,
                          hipStream_t s);
// f16 -> f32 widening of a vector (scales).
int launch_f16_to_f32(const void* src, float* dst, int64_t n, hipStream_t s);
// 64-bit content hash of a byte range (order-dependent, deterministic).
int launch_hash64(const void* src, int64_t bytes, uint64_t* out_dev, hipStream_t s);
// Adds to *count_dev the number of 4-byte words (and tail bytes) in which
// two 16-byte aligned ranges differ.
int launch_diff_bytes(const void* a, const void* b, int64_t bytes, unsigned* count_dev, hipStream_t s);
// Seeded uniform fill of n elements of type dt: integers in [lo, hi] for
// DT_I8, U[lo, hi) rounded to the type otherwise.
int launch_fill_uniform(void* dst, int64_t n, int dt, float lo, float hi, uint64_t seed, hipStream_t s);
// Adds to *count_dev the elements where |got - want| > atol + rtol |want|
// (or either is not finite), for DT_F16 / DT_BF16 / DT_F32 arrays.
int launch_count_far(const void* got, const void* want, int64_t n, int dt, float rtol, float atol,
                     unsigned* count_dev, hipStream_t s);

}  // namespace hx
