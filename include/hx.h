/*
 * hx.h -- C ABI of libhxmi, the MI355X (gfx950) implementation of the
 * hexagon-mlir hot path: the weight-resident tiled matmul (f16/bf16 and
 * int8), the W8A16 decode GEMV, the softmax / RMSNorm / LayerNorm row
 * reductions, the SwiGLU FFN composition, and the kernel-config surface the
 * tile autotuner searches.
 *
 * Reference paths below are relative to the hexagon-mlir checkout;
 * QHB = qcom_hexagon_backend.
 *
 * Conventions (all entry points):
 *   - Tensors are MLIR-style strided memref descriptors (hx_memref2d /
 *     hx_memref1d), field for field the MemRefDescriptor<T,N> the
 *     reference's compiled kernels receive (test/utils/dsp/include/
 *     common.h:15-21: allocated, aligned, offset, sizes[N], strides[N];
 *     built by Tensor::toMemRefDesc, tensor.h:73-90).
 *     Strides and offsets are in elements.  The innermost stride must be 1;
 *     the outer stride may exceed the row length (the multi-span output ABI
 *     of test/python/triton/test_matmul_multispan.py:71-78).
 *   - Data pointers are device pointers.  The caller owns every tensor; the
 *     library owns registered weights and a per-stream workspace.
 *   - Work is enqueued on `stream` (NULL = the null stream); no entry point
 *     synchronizes the device except hx_weight_register, hx_weight_release
 *     (of the last reference) and hx_tune.
 *   - Return value: HX_OK or a negative HX_ERR_*; hx_last_error() returns a
 *     thread-local message for the last failure.  Failures are closed: there
 *     is no silent fallback to another arithmetic path (the reference aborts
 *     on allocation failure, QHB/bin/runtime/include/HexagonCAPI.h:21-25;
 *     here the caller gets the code instead).
 *   - Safe to call from several host threads on distinct streams.
 */
#ifndef HX_H
#define HX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HX_ABI_VERSION 1

/* Same tag as hipStream_t, so a hipStream_t converts without a cast. */
typedef struct ihipStream_t* hx_stream_t;

/* Element types (the reference's admitted matmul dtypes are f16/f32 on HMX,
 * QHB/include/hexagon/Dialect/Hmx/IR/HmxDType.h:59-75; int8 runs on the HVX
 * linalg path, QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:169-196). */
enum { HX_F16 = 1, HX_BF16 = 2, HX_F32 = 3, HX_I8 = 4, HX_I32 = 5 };

/* Orientation of a right-hand operand / weight.  KN is linalg.matmul's
 * [K, N]; NK is the transposed source [N, K] that hmx.pack_weight accepts
 * with src_transposed (QHB/include/hexagon/Dialect/Hmx/IR/HmxOps.td:259-266)
 * and the layout the kernels consume directly. */
enum { HX_LAYOUT_KN = 0, HX_LAYOUT_NK = 1 };

enum {
    HX_OK = 0,
    HX_ERR_ARG = -1,         /* null / malformed argument */
    HX_ERR_SHAPE = -2,       /* operand shapes do not agree */
    HX_ERR_DTYPE = -3,       /* dtype combination not supported */
    HX_ERR_LAYOUT = -4,      /* innermost stride != 1, bad outer stride */
    HX_ERR_HIP = -5,         /* a HIP runtime call failed */
    HX_ERR_NOMEM = -6,       /* device allocation failed */
    HX_ERR_UNSUPPORTED = -7, /* valid request outside what is implemented */
    HX_ERR_HANDLE = -8,      /* unknown or released weight handle */
    HX_ERR_NODEVICE = -9     /* no HIP device visible */
};

typedef struct hx_memref2d {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[2];
    int64_t strides[2];
} hx_memref2d;

typedef struct hx_memref1d {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[1];
    int64_t strides[1];
} hx_memref1d;

/* Rank-4 descriptor ([Z][H][N][D] attention operands), same field meaning. */
typedef struct hx_memref4d {
    void* allocated;
    void* aligned;
    int64_t offset;
    int64_t sizes[4];
    int64_t strides[4];
} hx_memref4d;

/* ---------------------------------------------------------------------- */
/* Library state                                                           */
/* ---------------------------------------------------------------------- */

/* Initialise per-device state for the current HIP device.  Optional: every
 * entry point initialises lazily.  Replaces the runtime's power/HVX/HMX
 * acquire (QHB/bin/runtime/src/HexagonAPI.cpp:160-261). */
int hx_init(void);
const char* hx_last_error(void);
/* Identity of this build (compiler, arch, source digest); part of every
 * tuned-config cache key, as tuning_key_int is in QHB/backend/hmx_search.py:
 * 416-452. */
const char* hx_build_id(void);

/* ---------------------------------------------------------------------- */
/* Matmul family                                                           */
/* ---------------------------------------------------------------------- */

/* C = A . B  (overwrite), or C = A . B * col_scale + residual.
 *   a        [M, K]  f16 or bf16 (or f32, see below)
 *   b        [K, N] (HX_LAYOUT_KN) or [N, K] (HX_LAYOUT_NK); same dtype as
 *            a, or int8 with a = f16 (W8A16: int8 widened exactly to f16)
 *   f32 a or b: quantised to f16 before the product, (x + 0) rounded to
 *            nearest even (-0 becomes +0, beyond 65504 infinity), as the
 *            reference's f32 pack leaves and host prepack do
 *            (QHB/bin/runtime/hmx/src/HMXLayout.c:257-340;
 *            QHB/backend/hmx_weight_prepack.py:185-212); f32 a pairs with
 *            f32, f16 or int8 b, f32 b with f16 or f32 a
 *   col_scale NULL or [N] f32/f16: per-output-channel scale applied to the
 *            binary32 accumulator (the HMX conversion state's per-channel
 *            Scale, QHB/bin/runtime/hmx/src/HMXAPI.c:15-27, 39-44)
 *   residual NULL or [M, N] f16/bf16/f32, added after the scale
 *   c        [M, N] f16, bf16 or f32; one rounding from binary32
 * Replaces: linalg.matmul -> hmx.matmul (write-only, empty init) and the
 * residual/widening read-out (QHB/lib/Dialect/Hmx/Transforms/
 * MatmulToHmxPass.cpp:1-48, 100-121, 1369-1470; HmxOps.td:47-110,
 * 362-430; the leaves hmx_mma_f16 / hmx_acc_store_f16 / hmx_unpack_acc_f32,
 * QHB/bin/runtime/hmx/include/HMXAPI.h:66-80, 217-230). */
int hx_matmul(const hx_memref2d* a, int a_dtype,
              const hx_memref2d* b, int b_dtype, int b_layout,
              const hx_memref1d* col_scale, int scale_dtype,
              const hx_memref2d* residual, int residual_dtype,
              hx_memref2d* c, int c_dtype, hx_stream_t stream);

/* int8 x int8 -> int32, exact: C[i][j] = sum_k sext(A[i][k]) * sext(B[k][j]).
 *   c_dtype HX_I32: the int32 product itself.
 *   c_dtype HX_F16: RNE_f16(((float)C[i][j] * row_scale[i]) * col_scale[j]),
 *                   binary32, in that order; either scale may be NULL (1).
 * Scales are f32.  Replaces linalg.matmul(i8, i8 -> i32) as lowered by
 * ScheduleMatmulForHVX (QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:
 * 48-199), the path matmul-to-hmx leaves int8 on (`unsupported-dtype`,
 * QHB/include/hexagon/Dialect/Hmx/Transforms/HmxTarget.h:198-200). */
int hx_gemm_i8(const hx_memref2d* a, const hx_memref2d* b, int b_layout,
               const hx_memref1d* row_scale, const hx_memref1d* col_scale,
               hx_memref2d* c, int c_dtype, hx_stream_t stream);

/* W8A16 decode GEMV / skinny GEMM, M <= 16 (any M is accepted; M > 16 runs
 * the MFMA GEMM with the same contract):
 *   Y[m][n] = RNE_f16( (sum_k X[m][k] * W[k][n]) * scale[n] ),
 *   X [M, K] f16, W int8 [K, N] (KN) or [N, K] (NK), scale [N] f16/f32.
 * Replaces the HVX dequant-generic + matmul that skinny shapes take
 * (HmxTarget.h:100 `min-rows`, :208-216 `tile-alignment`;
 * ScheduleMatmulForHVXPass.cpp:169-196). */
int hx_gemv_w8a16(const hx_memref2d* x, const hx_memref2d* w, int w_layout,
                  const hx_memref1d* scale, int scale_dtype,
                  hx_memref2d* y, hx_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Row reductions over the last dimension (f16, bf16 or f32 in and out,   */
/* binary32 inside, one rounding)                                          */
/* ---------------------------------------------------------------------- */

/* y = exp(x - max) * (1 / sum exp(x - max)).
 * Replaces the softmax generic chain (docs/tutorials/torch-mlir/
 * softmax.md:178-226; test/python/triton/test_softmax.py:41-69) as fused by
 * HexagonFusion and VectorRowReduce (QHB/lib/Conversion/LinalgToLLVM/
 * FusionPass.cpp:223, VectorRowReducePass.cpp:1-31) with DivToMul
 * (QHB/lib/Transforms/DivToMulOptimizationPass.cpp:9-18). */
/* Row kernels (softmax, RMSNorm, LayerNorm) hold a row in registers up to
 * 4096 16-byte vectors, i.e. 16384 binary32 or 32768 f16/bf16 elements per
 * row (softmax over 16-byte-aligned rows, 64 rows or more: up to 16384
 * vectors), and stream longer rows in two passes (the two-phase online
 * softmax of test/python/triton/test_online_softmax.py:28-78, and its
 * counterparts for the norms), with rows x (at most 64 segments) x 16 bytes
 * of statistics in the stream workspace. */
int hx_softmax(const hx_memref2d* x, hx_memref2d* y, int dtype, hx_stream_t stream);

/* y = x * rsqrt(sum(x^2)/N + eps) * gamma   (gamma may be NULL).
 * Replaces test/python/triton/test_rms_norm.py:34-59 after FastInverse
 * (QHB/lib/Transforms/FastInversePass.cpp:97-140). */
int hx_rmsnorm(const hx_memref2d* x, const hx_memref1d* gamma, float eps,
               hx_memref2d* y, int dtype, hx_stream_t stream);

/* y = (x - mean) * rstd * w + b; mean / rstd (f32 [rows]) are written when
 * non-NULL.  w, b may be NULL.  Replaces test/python/triton/
 * test_layer_norm.py:39-79 (mean and rstd stored as at :70-72). */
int hx_layernorm(const hx_memref2d* x, const hx_memref1d* w, const hx_memref1d* b,
                 float eps, hx_memref2d* y, hx_memref1d* mean, hx_memref1d* rstd,
                 int dtype, hx_stream_t stream);

/* out = RNE(silu(g) * u), silu(g) = g / (1 + exp(-g)); f16 only.
 * The SiLU of test/python/triton/test_silu.py applied as the SwiGLU gate. */
int hx_silu_mul(const hx_memref2d* g, const hx_memref2d* u, hx_memref2d* out,
                int dtype, hx_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Resident weights                                                        */
/* ---------------------------------------------------------------------- */

typedef struct hx_weight* hx_weight_t;

/* Register a weight once: the library builds its K-contiguous device image
 * ([N, K]) and f32 per-channel scales, keyed by content (a second
 * registration of identical bytes, shape, dtype and scales returns the same
 * handle with its reference count raised).  w_dtype HX_I8 (scale required,
 * [N] f16/f32), HX_F16, HX_BF16 (scale optional), or HX_F32: quantised to
 * f16 as hx_matmul quantises f32 operands and held as an f16 weight.
 * Synchronizes `stream`.
 * Replaces the resident-weight ABI hexagon_runtime_weight_resident_v2
 * (QHB/bin/runtime/include/HexagonCAPI.h:39-57) together with the host
 * pre-pack and its content-hash cache (QHB/backend/hmx_weight_prepack.py:
 * 124-212) and WeightResidentPass (QHB/lib/Dialect/Hmx/Transforms/
 * WeightResidentPass.cpp:1-60). */
int hx_weight_register(const hx_memref2d* w, int w_dtype, int w_layout,
                       const hx_memref1d* scale, int scale_dtype,
                       hx_stream_t stream, hx_weight_t* out);
/* Drop one reference; the image is freed when the count reaches zero. */
int hx_weight_release(hx_weight_t w);
int hx_weight_info(hx_weight_t w, int64_t* k, int64_t* n, int* dtype,
                   uint64_t* content_hash, int* refcount);

/* Y = X . W * scale (+ residual) with a registered weight.  X [M, K] f16
 * (bf16 for a bf16 weight), Y [M, N] f16/bf16/f32.  Skinny products (int8
 * weights M <= 32, and up to 64 where the GEMV's four row blocks beat the
 * GEMM: 129..256 column tiles of 16 with K >= 8192, or 641..768 tiles up to
 * M = 48; f16 / bf16 M <= 16, or M <= 32 with N >= 2048, or M <= 64 on
 * 641..768 tiles with K >= 4096) run the decode GEMV
 * on the weight's fragment-packed copy (registration keeps it beside the
 * [N, K] image: twice the weight's bytes), larger M the MFMA GEMM. */
int hx_matmul_resident(const hx_memref2d* x, int x_dtype, hx_weight_t w,
                       const hx_memref2d* residual, int residual_dtype,
                       hx_memref2d* y, int y_dtype, hx_stream_t stream);

/* Llama-style SwiGLU FFN block on registered int8 weights:
 *   h = RMSNorm(x, gamma, eps); a = silu(h.Wg*sg) * (h.Wu*su); y = a.Wd*sd
 * with fp16 rounding after each linalg op (RMSNorm out, gate, up, SiLU*mul,
 * down).  x [T, H] f16, Wg/Wu [H, I], Wd [I, H] (as registered), y [T, H].
 * The gate and up GEMMs share one kernel whose epilogue applies SiLU*mul. */
int hx_swiglu_ffn(const hx_memref2d* x, const hx_memref1d* gamma, float eps,
                  hx_weight_t w_gate, hx_weight_t w_up, hx_weight_t w_down,
                  hx_memref2d* y, hx_stream_t stream);

/* Size of the fixed per-GPU scratch of hx_swiglu_ffn_noalloc (32 MiB). */
#define HX_NOALLOC_SCRATCH_BYTES (32 << 20)

/* hx_swiglu_ffn that allocates nothing.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments and bit-identical result as hx_swiglu_ffn; the RMSNorm
 * output, the gate/up/SiLU*mul intermediates and the down projection's
 * K-split partials live in a fixed device array of HX_NOALLOC_SCRATCH_BYTES
 * that each GPU the library runs on holds until the process ends, instead
 * of the stream workspace.  The call makes no hipMalloc or hipFree.  It
 * needs T*(H + I)*2 bytes for T > 32 tokens (at most T*(H + 3 I)*2 for T <= 32, the
 * decode path), plus T*H*4 per K part when the down projection's
 * configuration splits K (on the decode path T*N*4 per part, N = I or H,
 * for the decode GEMVs whose configuration splits K; 256-byte aligned
 * each), out of the array
 * less its last 64 KiB (the split decode GEMV's counters, zero between
 * calls); a shape that needs more returns HX_ERR_UNSUPPORTED before
 * anything is enqueued.  Every call on one GPU shares its array: calls that
 * overlap on one GPU race. */
int hx_swiglu_ffn_noalloc(const hx_memref2d* x, const hx_memref1d* gamma, float eps,
                          hx_weight_t w_gate, hx_weight_t w_up, hx_weight_t w_down,
                          hx_memref2d* y, hx_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Kernel configurations (the autotuner's search space)                    */
/* ---------------------------------------------------------------------- */

/* Kernel families. */
enum {
    HX_OP_GEMM_I8 = 1,      /* hx_gemm_i8 */
    HX_OP_MATMUL_F16 = 2,   /* hx_matmul f16 x f16 */
    HX_OP_MATMUL_BF16 = 3,  /* hx_matmul bf16 x bf16 */
    HX_OP_MATMUL_W8 = 4,    /* f16 x int8 GEMM (M > 16) */
    HX_OP_SWIGLU_W8 = 5,    /* fused gate/up GEMM of hx_swiglu_ffn */
    HX_OP_GEMV_W8 = 6,      /* W8A16 decode GEMV (M <= 16) */
    HX_OP_GEMV_F16 = 7,     /* f16 x f16 decode GEMV (M <= 16), same configs as 6 */
    HX_OP_GEMV_BF16 = 8,    /* bf16 x bf16 decode GEMV (M <= 16), same configs as 6 */
    HX_OP_SOFTMAX = 9,      /* hx_softmax; row families: m = rows, n = cols, k = dtype */
    HX_OP_RMSNORM = 10,     /* hx_rmsnorm */
    HX_OP_LAYERNORM = 11    /* hx_layernorm */
};

/* One compiled configuration.  GEMM families fill bm/bn/bk (K elements per
 * LDS stage)/waves_m/waves_n/lds_stages (K stages resident in LDS: 2 or 3)/
 * split_k (K parts, merged inside the kernel by the last part of each
 * tile to finish, or by a merge kernel when the tiles outnumber the split
 * counters; 1: none); the GEMV
 * families fill col_tiles (16-column tiles per workgroup), waves_m (waves
 * splitting K inside a workgroup) and split_k (workgroups splitting K per
 * group of col_tiles tiles, the last of them to finish adding the parts;
 * 1: none).  The row families (softmax, RMSNorm, LayerNorm) fill col_tiles
 * with the workgroups per CU of the streaming form ("stream_N": a grid of
 * N workgroups per CU walks the rows, gamma / beta resident, two rows in
 * flight per workgroup) or 0 ("row": one row per workgroup); waves_m is the
 * streaming form's waves per row.  Every row configuration computes the
 * same bits; rows that the streaming form does not take (under 4 KiB, over
 * 64 KiB, unaligned) run "row" whatever is pinned.  hx_tune does not time
 * row families: pin them with hx_config_select.
 * Replaces the (BM, BN, BK) tile space of enumerate_tile_configs
 * (QHB/backend/hmx_search.py:246-332), widened to the knobs that matter on
 * gfx950. */
typedef struct hx_kernel_config {
    int32_t op;
    int32_t index;
    int32_t bm, bn, bk;
    int32_t waves_m, waves_n;
    int32_t lds_stages;
    int32_t split_k;
    int32_t col_tiles;
    int32_t lds_bytes;
    char name[40];
} hx_kernel_config;

int hx_config_count(int op);
int hx_config_get(int op, int index, hx_kernel_config* out);
/* Pin configuration `index` for calls of family `op` with exactly this
 * (M, N, K) on the current device; index -1 removes the pin. */
int hx_config_select(int op, int64_t m, int64_t n, int64_t k, int index);
/* The configuration a call of this shape will run: the pinned one, else
 * the untuned default.  *index = -1 means the generic (any-alignment)
 * kernel. */
int hx_config_lookup(int op, int64_t m, int64_t n, int64_t k, int* index);
/* Persist the tuner's state: hx_config_pins_save writes the current
 * device's pins and canary references as text ("hx-pins/v2 <build id>",
 * then one "pin op m n k index name" line per pin and one "canary op q50_us"
 * line per family with a canary reference; NUL-terminated, *needed = size;
 * HX_ERR_ARG if cap is too small) and hx_config_pins_load restores them in
 * another process.  Text from another build is refused (a config index
 * means nothing across builds), as is any line whose index does not name
 * the same config; a refused load changes nothing.  Replaces the
 * tuned-config cache of QHB/backend/hmx_search.py (keyed by build
 * fingerprints, tuning_key_int :416-452) and the canary record the next
 * round is judged against (:1292-1368). */
int hx_config_pins_save(char* buf, size_t cap, size_t* needed);
int hx_config_pins_load(const char* text);

/* ---------------------------------------------------------------------- */
/* Autotuning                                                              */
/* ---------------------------------------------------------------------- */

/* Status of one configuration in a tuning round. */
enum {
    HX_TUNE_TIMED = 0,          /* timed; q50/q20/q80 hold its per-launch times */
    HX_TUNE_REFUSED = 1,        /* not legal at this shape; `reason` says why */
    HX_TUNE_LAUNCH_FAILED = 2,  /* a launch or its timing failed: scored infinite */
    HX_TUNE_WRONG = 3           /* its first launch disagreed with the reference
                                   kernel: scored infinite after one launch */
};

/* The canary: the family's untuned default on a small fixed shape, timed
 * after the sweep and judged against the family's previous valid round. */
enum {
    HX_CANARY_BASELINE = 0,     /* no earlier reading: this one becomes the reference */
    HX_CANARY_STEADY = 1,       /* within its gate of the reference */
    HX_CANARY_DRIFT = 2,        /* moved by more than its gate: the round is void */
    HX_CANARY_FAILED = 3        /* could not be timed: the round is void */
};

typedef struct hx_tune_options {
    int32_t reps;               /* repetitions per configuration; 0 = 3 */
    int32_t min_iters;          /* launches per repetition = clamp(budget / one */
    int32_t max_iters;          /*   launch, min, max); 0 = 5 and 1000 */
    double budget_us;           /* device time aimed at per repetition; 0 = 2e6 */
    double canary_reference_us; /* > 0: judge the canary against this median;
                                   0: against the family's held reference (the
                                   last valid round, or hx_config_pins_load);
                                   < 0: no reference (the round sets one) */
    int32_t pin;                /* pin the champion when the round is valid */
    uint64_t seed;              /* synthetic operand seed; 0 = a fixed default */
} hx_tune_options;

typedef struct hx_tune_entry {
    int32_t index;              /* family configuration index (hx_config_get) */
    int32_t status;             /* HX_TUNE_* */
    double q50_us, q20_us, q80_us;  /* quantiles over the repetitions of the
                                       mean per-launch device time (inf unless
                                       timed) */
    char reason[24];            /* "timed", or the refusal / failure */
} hx_tune_entry;

#define HX_TUNE_MAX_ENTRIES 64

typedef struct hx_tune_report {
    int32_t op;
    int64_t m, n, k;
    int32_t iters;              /* launches per repetition (largest used) */
    int32_t control_index;      /* the untuned default: the control arm */
    int32_t best_index;         /* the fastest timed configuration, or -1 */
    int32_t champion_index;     /* best when it beats the control by more than
                                   the gate (or no control was timed), else the
                                   control; -1 when nothing was timed */
    double control_q50_us, best_q50_us;
    double margin;              /* (control - best) / control */
    double gate;                /* max(3 * CV, 0.15), CV = (q80 - q20) / q50 of
                                   the noisier of the two arms */
    int32_t canary_index;
    int64_t canary_m, canary_n, canary_k;
    int32_t canary_status;      /* HX_CANARY_* */
    double canary_q50_us, canary_reference_us;
    double canary_shift;        /* (canary - reference) / reference */
    double canary_gate;         /* max(3 * CV_canary, 0.15) */
    int32_t round_valid;        /* canary BASELINE or STEADY */
    int32_t pinned;             /* this call pinned the champion */
    int32_t n_entries;
    hx_tune_entry entries[HX_TUNE_MAX_ENTRIES];
} hx_tune_report;

/* Autotune family `op` at (m, n, k) on the current device: every compiled
 * configuration runs on synthetic seeded operands the call allocates
 * (weights of the decode families rotated over copies larger than the
 * 256 MB MALL), its first launch is checked against the generic kernel
 * (bit-equal for int8, within 1e-2 relative for floats), and it is timed
 * with HIP events on `stream` for `reps` repetitions.  The champion is the
 * fastest configuration if it beats the untuned default by more than the
 * gate, else the default.  The round is void when the canary drifted or
 * failed; a void round pins nothing and leaves every earlier pin in place.
 * A valid round becomes the family's canary reference.  Synchronizes
 * `stream`; allocates and frees device memory.  Replaces the tile search of
 * QHB/backend/hmx_search.py: enumerate_tile_configs / tile_verdict
 * (:246-332), hexagon_bench (:1109-1156), calibration_iters (:1159-1177),
 * quantile_spread_cv / champion_gate (:1254-1289) and the canary
 * (:1292-1368). */
int hx_tune(int op, int64_t m, int64_t n, int64_t k, const hx_tune_options* opt,
            hx_tune_report* out, hx_stream_t stream);

/* The decision of hx_tune alone, with no device work: from timed entries,
 * the control's configuration index, the canary's entry and a reference
 * median (<= 0: none), fill best/champion/margin/gate and the canary and
 * round fields of `out`. */
int hx_tune_decide(const hx_tune_entry* entries, int n, int control_index,
                   const hx_tune_entry* canary, double canary_reference_us,
                   hx_tune_report* out);

/* ---------------------------------------------------------------------- */
/* Scaled-dot-product attention                                            */
/* ---------------------------------------------------------------------- */

/* O = softmax(Q K^T * scale [, causal]) V per (z, h): q, o [Z][H][Nq][D],
 * k, v [Z][H][Nk][D] (innermost stride 1), dtype HX_F16 or HX_BF16, D 64 or
 * 128.  Scores and accumulation in binary32, online softmax in the exp2
 * domain (one pass over K/V, no Nq x Nk intermediate); causal masks key j
 * for query i when j > i.  Replaces the FlashAttention forward the Triton
 * front end compiles (test/python/triton/test_flash_attention.py:
 * _attn_fwd_inner, attention_fwd_kernel) and its online-softmax recurrence
 * (test/python/triton/test_online_softmax.py:28-78); same arithmetic
 * (qk_scale = scale * log2 e, p = exp2(qk * qk_scale - m), O = acc / l). */
int hx_attention(const hx_memref4d* q, const hx_memref4d* k, const hx_memref4d* v, hx_memref4d* o,
                 float scale, int causal, int dtype, hx_stream_t stream);

/* ---------------------------------------------------------------------- */
/* Plan manifest                                                           */
/* ---------------------------------------------------------------------- */

/* While enabled, every matmul-family call (hx_matmul, hx_gemm_i8,
 * hx_gemv_w8a16, hx_matmul_resident, the GEMMs of hx_swiglu_ffn) records the
 * plan it ran -- kernel path ("mfma-tiled", "mfma-generic", "gemv",
 * "gemv-packed"), tile configuration and whether the tuner pinned it, the
 * reason ("selected-aligned", "min-rows", or the fast-path precondition that
 * failed), and how the weight was supplied -- one record per distinct
 * decision with a call count.  Replaces the per-matmul semantic manifest
 * `hmx.kernel_manifest` with its plan/reason vocabulary
 * (QHB/include/hexagon/Dialect/Hmx/Transforms/HmxManifest.h:41, 81-110) and
 * its JSON export (QHB/backend/utils.py:1055-1196); here the decisions are
 * made per call at run time, so they are recorded at run time.
 * hx_manifest_enable returns the previous state.  hx_manifest_json writes
 * a NUL-terminated JSON document {"schema": "hx.kernel_manifest/v1",
 * "build": ..., "records": [...]} into buf and sets *needed to its size;
 * HX_ERR_ARG (with *needed set) when cap is too small. */
int hx_manifest_enable(int on);
int hx_manifest_clear(void);
int hx_manifest_json(char* buf, size_t cap, size_t* needed);

/* ---------------------------------------------------------------------- */
/* Clock probe                                                             */
/* ---------------------------------------------------------------------- */

/* A measurement hook with no counterpart in the reference (whose profiler
 * reads the Hexagon cycle counters, QHB/backend/hmx_search.py:1109-1156
 * "PerfPcycles"): it reports the shader clock MFMA-bound kernels actually
 * ran at, which on MI355X varies with the operands' data.  While enabled on
 * the current device, every workgroup of the tiled GEMM kernels (hx_gemm_i8,
 * hx_matmul, hx_matmul_resident beyond the decode sizes, the GEMMs of
 * hx_swiglu_ffn) adds its elapsed shader-clock cycles (s_memtime) and
 * constant-rate ticks (s_memrealtime) to a per-device pair of counters.
 * hx_clock_probe(1) allocates (first use) and zeroes the counters and waits
 * for the device; hx_clock_probe(0) stops the stamping.  hx_clock_read waits
 * for the device and returns the mean clock over the stamped workgroups in
 * MHz, the summed workgroup time in microseconds and the workgroup count. */
int hx_clock_probe(int enable);
int hx_clock_read(double* mhz, double* workgroup_us, long long* workgroups);

#ifdef __cplusplus
}
#endif

#endif /* HX_H */
