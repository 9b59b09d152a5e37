/*
 * hx_oracle.c -- CPU restatement of the linalg semantics the Hexagon-MLIR
 * backend lowers for the matmul / softmax / RMSNorm / LayerNorm hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library and the timed CPU baseline of bench.py.  Nothing in the product
 * path links, loads or calls it; the product fails loudly when its HIP
 * library is missing instead of falling back here.
 *
 * Every function names the reference file:line whose semantics it follows
 * (paths relative to the hexagon-mlir checkout, QHB = qcom_hexagon_backend).
 * Each function is pinned by tests/test_oracle.py against numpy / torch-CPU
 * library routines, closed forms, invariants and brute force; see the table
 * in that file's docstring.
 *
 * Rounding model: all floating-point arithmetic is IEEE binary32 with
 * round-to-nearest-even, no contraction (-ffp-contract=off), sequential
 * accumulation in the reference's loop order.  Narrowing to fp16 / bf16 is
 * round-to-nearest-even with overflow to infinity.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

enum { HXO_F16 = 1, HXO_BF16 = 2, HXO_F32 = 3, HXO_I8 = 4, HXO_I32 = 5 };

/* ------------------------------------------------------------------------ */
/* Narrowing / widening conversions                                          */
/* ------------------------------------------------------------------------ */

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* binary32 -> binary16, round to nearest even.  The reference's f32 pack
 * quantises the same way (QHB/bin/runtime/hmx/src/HMXLayout.c:257-340,
 * QHB/backend/hmx_weight_prepack.py:185-212 "f32 -> f16 RNE"). */
uint16_t hxo_f32_to_f16(float f)
{
    uint32_t x = bits_of(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u)                       /* NaN: quiet, keep top payload */
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x477ff000u)                      /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    if (a >= 0x38800000u) {                    /* normal binary16 result */
        uint32_t odd = (a >> 13) & 1u;
        a -= 0x38000000u;                      /* rebias exponent 127 -> 15 */
        a += 0x0fffu + odd;                    /* RNE on the 13 dropped bits */
        return (uint16_t)(sign | (a >> 13));
    }
    /* subnormal or zero: let the FPU's RNE addition align the mantissa.
     * 0.5f has exponent 126 = 127-15+23-10+1, so the sum's low 10 bits are
     * the binary16 subnormal mantissa (or 0x400 when it rounds up to 2^-14). */
    float g = float_of(a) + 0.5f;
    return (uint16_t)(sign | (bits_of(g) - 0x3f000000u));
}

float hxo_f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f)
        return float_of(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        /* subnormal: m * 2^-24 is exact in binary32 */
        float v = (float)m * float_of(0x33800000u);
        return sign ? -v : v;
    }
    return float_of(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t hxo_f32_to_bf16(float f)
{
    uint32_t x = bits_of(f);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x40u);   /* quiet NaN */
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float hxo_bf16_to_f32(uint16_t h) { return float_of((uint32_t)h << 16); }

void hxo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = hxo_f32_to_f16(in[i]);
}
void hxo_f16_to_f32_array(const uint16_t* in, float* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = hxo_f16_to_f32(in[i]);
}
void hxo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n)
{
    for (int64_t i = 0; i < n; ++i) out[i] = hxo_f32_to_bf16(in[i]);
}

static inline float load_elem(const void* p, int dtype, int64_t i)
{
    switch (dtype) {
    case HXO_F16: return hxo_f16_to_f32(((const uint16_t*)p)[i]);
    case HXO_BF16: return hxo_bf16_to_f32(((const uint16_t*)p)[i]);
    case HXO_I8: return (float)((const int8_t*)p)[i];
    case HXO_I32: return (float)((const int32_t*)p)[i];
    default: return ((const float*)p)[i];
    }
}

static inline void store_elem(void* p, int dtype, int64_t i, float v)
{
    switch (dtype) {
    case HXO_F16: ((uint16_t*)p)[i] = hxo_f32_to_f16(v); break;
    case HXO_BF16: ((uint16_t*)p)[i] = hxo_f32_to_bf16(v); break;
    default: ((float*)p)[i] = v; break;
    }
}

/* ------------------------------------------------------------------------ */
/* int8 x int8 -> int32 GEMM                                                 */
/* ------------------------------------------------------------------------ */

/* C[i][j] = sum_k sext(A[i][k]) * sext(B[k][j]) in int32.
 *
 * Follows ScheduleMatmulForHVX (QHB/lib/Transforms/ScheduleMatmulForHVXPass.cpp:
 * 169-196): linalg.matmul generalised to a linalg.generic with the (i,k,j)
 * loop order and body out + extsi(a)*extsi(b).  Integer addition is exact and
 * associative mod 2^32, so the loop order does not change a single bit; it
 * is kept because this loop is also the timed CPU baseline.
 * B is [K][N] with row stride ldb, or [N][K] (ldb) when b_trans != 0. */
void hxo_gemm_i8_i32(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                     int b_trans, int32_t* C, int64_t ldc,
                     int64_t M, int64_t N, int64_t K)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
        int32_t* c = C + i * ldc;
        const int8_t* a = A + i * lda;
        if (!b_trans) {
            for (int64_t j = 0; j < N; ++j) c[j] = 0;
            for (int64_t k = 0; k < K; ++k) {
                const int32_t av = a[k];
                const int8_t* b = B + k * ldb;
                for (int64_t j = 0; j < N; ++j) c[j] += av * (int32_t)b[j];
            }
        } else {
            for (int64_t j = 0; j < N; ++j) {
                const int8_t* b = B + j * ldb;
                int32_t s = 0;
                for (int64_t k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
                c[j] = s;
            }
        }
    }
}

/* Dequantise an int32 product to fp16 with per-row and per-column fp32
 * scales: out = RNE_f16(((float)C[i][j] * sa[i]) * sb[j]).  The per-channel
 * scale is the HMX conversion state's Scale field (QHB/bin/runtime/hmx/src/
 * HMXAPI.c:15-27, 39-44; the reference always loads identity there); the
 * order (row scale first, then column scale, binary32) is this build's
 * definition and the GPU epilogue reproduces it bit for bit.
 * sa / sb may be NULL (scale 1). */
void hxo_dequant_i32_f16(const int32_t* C, int64_t ldc, const float* sa,
                         const float* sb, uint16_t* out, int64_t ldo,
                         int64_t M, int64_t N)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < M; ++i) {
        const float ra = sa ? sa[i] : 1.0f;
        for (int64_t j = 0; j < N; ++j) {
            float t = (float)C[i * ldc + j] * ra;
            if (sb) t = t * sb[j];
            out[i * ldo + j] = hxo_f32_to_f16(t);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Floating-point matmul (f16 / bf16 / f32 operands, or int8 weights)        */
/* ------------------------------------------------------------------------ */

/* out[i][j] = round_cdt( acc[i][j] * scale_n[j] + R[i][j] ),
 * acc[i][j] = sum_k A[i][k] * B[k][j] accumulated in binary32, (i,k,j) order.
 *
 * Semantics of linalg.matmul as MatmulToHmx treats it
 * (QHB/lib/Dialect/Hmx/Transforms/MatmulToHmxPass.cpp:1-48, 100-121): an
 * empty init is an overwrite, a non-empty init C is added as a residual
 * (the fused unpack_acc_f32 + residual read-out, QHB/bin/runtime/hmx/src/
 * HMXLayout.c:868-999).  B may be int8 (W8A16): the dequant generic sitofp
 * is exact for |w| <= 127, and the per-output-channel scale multiplies the
 * fp32 accumulator (the HMX per-channel Scale hook, HMXAPI.c:15-27).
 * scale_n and R may be NULL.  B is [K][N] (ldb) or [N][K] when b_trans. */
void hxo_matmul(const void* A, int a_dtype, int64_t lda,
                const void* B, int b_dtype, int64_t ldb, int b_trans,
                const float* scale_n, const void* R, int r_dtype, int64_t ldr,
                void* C, int c_dtype, int64_t ldc,
                int64_t M, int64_t N, int64_t K)
{
#pragma omp parallel
    {
        /* per-thread fp32 accumulator row */
        float acc_stack[4096];
        float* acc = acc_stack;
        float* heap = 0;
        if (N > 4096) {
            heap = (float*)__builtin_malloc((size_t)N * sizeof(float));
            acc = heap;
        }
#pragma omp for schedule(static)
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = 0; j < N; ++j) acc[j] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float a = load_elem(A, a_dtype, i * lda + k);
                if (!b_trans) {
                    for (int64_t j = 0; j < N; ++j)
                        acc[j] = acc[j] + a * load_elem(B, b_dtype, k * ldb + j);
                } else {
                    for (int64_t j = 0; j < N; ++j)
                        acc[j] = acc[j] + a * load_elem(B, b_dtype, j * ldb + k);
                }
            }
            for (int64_t j = 0; j < N; ++j) {
                float v = acc[j];
                if (scale_n) v = v * scale_n[j];
                if (R) v = v + load_elem(R, r_dtype, i * ldr + j);
                store_elem(C, c_dtype, i * ldc + j, v);
            }
        }
        if (heap) __builtin_free(heap);
    }
}

/* hxo_matmul with the threads splitting the output columns instead of the
 * rows, for products with fewer rows than host threads (the decode GEMV's
 * M = 1..16).  Each output element is still the sum over k in increasing
 * order, accumulated in binary32, then scaled and added to the residual, so
 * the result is bit-identical to hxo_matmul's (pinned by test_oracle.py).
 * Column blocks of 64 keep a thread's accumulators in a stack row. */
void hxo_matmul_ncols(const void* A, int a_dtype, int64_t lda,
                      const void* B, int b_dtype, int64_t ldb, int b_trans,
                      const float* scale_n, const void* R, int r_dtype, int64_t ldr,
                      void* C, int c_dtype, int64_t ldc,
                      int64_t M, int64_t N, int64_t K)
{
    const int64_t JB = 64;
    const int64_t nblk = (N + JB - 1) / JB;
#pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < nblk; ++blk) {
        float acc[64];
        const int64_t j0 = blk * JB;
        const int64_t j1 = j0 + JB < N ? j0 + JB : N;
        for (int64_t i = 0; i < M; ++i) {
            for (int64_t j = j0; j < j1; ++j) acc[j - j0] = 0.0f;
            for (int64_t k = 0; k < K; ++k) {
                const float a = load_elem(A, a_dtype, i * lda + k);
                if (!b_trans) {
                    for (int64_t j = j0; j < j1; ++j)
                        acc[j - j0] = acc[j - j0] + a * load_elem(B, b_dtype, k * ldb + j);
                } else {
                    for (int64_t j = j0; j < j1; ++j)
                        acc[j - j0] = acc[j - j0] + a * load_elem(B, b_dtype, j * ldb + k);
                }
            }
            for (int64_t j = j0; j < j1; ++j) {
                float v = acc[j - j0];
                if (scale_n) v = v * scale_n[j];
                if (R) v = v + load_elem(R, r_dtype, i * ldr + j);
                store_elem(C, c_dtype, i * ldc + j, v);
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Row reductions                                                            */
/* ------------------------------------------------------------------------ */

/* Numerically stable softmax over the last dimension, binary32 internally,
 * one rounding to the output dtype:
 *   m = max_j x_j ;  e_j = exp(x_j - m) ;  s = sum_j e_j ;  y_j = e_j * (1/s)
 * Decomposition: docs/tutorials/torch-mlir/softmax.md:178-226 (max-reduce,
 * sub, exp, sum-reduce, div) and test/python/triton/test_softmax.py:59-68;
 * the divide is a multiply by the reciprocal after DivToMul
 * (QHB/lib/Transforms/DivToMulOptimizationPass.cpp:9-18).  The reduction
 * folds its init into one value per row (QHB/lib/Conversion/LinalgToLLVM/
 * VectorRowReducePass.cpp:17-28).  exp is libm expf; the reference's is the
 * Hexagon SDK's qhmath_hvx_exp (not vendored), pinned only by the reference
 * test's tolerance against torch. */
void hxo_softmax(const void* x, void* y, int dtype, int64_t rows, int64_t cols,
                 int64_t ldx, int64_t ldy)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float m = -INFINITY;
        for (int64_t j = 0; j < cols; ++j) {
            float v = load_elem(x, dtype, r * ldx + j);
            m = v > m ? v : m;
        }
        float s = 0.0f;
        for (int64_t j = 0; j < cols; ++j)
            s = s + expf(load_elem(x, dtype, r * ldx + j) - m);
        const float inv = 1.0f / s;
        for (int64_t j = 0; j < cols; ++j) {
            float e = expf(load_elem(x, dtype, r * ldx + j) - m);
            store_elem(y, dtype, r * ldy + j, e * inv);
        }
    }
}

/* RMSNorm: y = (x * rsqrt(sum(x^2)/N + eps)) * g, binary32 internally.
 * test/python/triton/test_rms_norm.py:34-59 computes x / sqrt(ms + eps) * g;
 * FastInverse rewrites x/sqrt(a) into x*rsqrt(a)
 * (QHB/lib/Transforms/FastInversePass.cpp:97-140), the form used here with
 * a correctly rounded 1/sqrtf.  gamma may be NULL (identity). */
void hxo_rmsnorm(const void* x, const void* gamma, float eps, void* y,
                 int dtype, int64_t rows, int64_t cols, int64_t ldx, int64_t ldy)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float ss = 0.0f;
        for (int64_t j = 0; j < cols; ++j) {
            float v = load_elem(x, dtype, r * ldx + j);
            ss = ss + v * v;
        }
        const float ms = ss / (float)cols;
        const float rs = 1.0f / sqrtf(ms + eps);
        for (int64_t j = 0; j < cols; ++j) {
            float v = load_elem(x, dtype, r * ldx + j) * rs;
            if (gamma) v = v * load_elem(gamma, dtype, j);
            store_elem(y, dtype, r * ldy + j, v);
        }
    }
}

/* LayerNorm, test/python/triton/test_layer_norm.py:39-79:
 *   mean = sum(x)/N ; d = x - mean ; var = sum(d^2)/N ;
 *   rstd = 1/sqrt(var + eps) ; y = d * rstd * w + b
 * mean / rstd (binary32, one per row) are written when non-NULL, as the
 * reference kernel stores them for the backward pass (:70-72).
 * w / b may be NULL (identity / zero). */
void hxo_layernorm(const void* x, const void* w, const void* b, float eps,
                   void* y, float* mean_out, float* rstd_out, int dtype,
                   int64_t rows, int64_t cols, int64_t ldx, int64_t ldy)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float s = 0.0f;
        for (int64_t j = 0; j < cols; ++j) s = s + load_elem(x, dtype, r * ldx + j);
        const float mean = s / (float)cols;
        float vs = 0.0f;
        for (int64_t j = 0; j < cols; ++j) {
            float d = load_elem(x, dtype, r * ldx + j) - mean;
            vs = vs + d * d;
        }
        const float var = vs / (float)cols;
        const float rstd = 1.0f / sqrtf(var + eps);
        if (mean_out) mean_out[r] = mean;
        if (rstd_out) rstd_out[r] = rstd;
        for (int64_t j = 0; j < cols; ++j) {
            float v = (load_elem(x, dtype, r * ldx + j) - mean) * rstd;
            if (w) v = v * load_elem(w, dtype, j);
            if (b) v = v + load_elem(b, dtype, j);
            store_elem(y, dtype, r * ldy + j, v);
        }
    }
}

/* SwiGLU gate: out = silu(g) * u = (g / (1 + exp(-g))) * u, binary32
 * internally, one rounding.  The SiLU form of test/python/triton/
 * test_silu.py (x * sigmoid(x)); used between the gate/up and down GEMMs of
 * the FFN composition. */
void hxo_silu_mul(const void* g, const void* u, void* out, int dtype,
                  int64_t rows, int64_t cols, int64_t ldg, int64_t ldu, int64_t ldo)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t j = 0; j < cols; ++j) {
            float gv = load_elem(g, dtype, r * ldg + j);
            float uv = load_elem(u, dtype, r * ldu + j);
            float s = gv / (1.0f + expf(-gv));
            store_elem(out, dtype, r * ldo + j, s * uv);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Scaled-dot-product attention                                              */
/* ------------------------------------------------------------------------ */

/* O = softmax(Q K^T * scale) V for one (z, h) slice per b < B:
 * q, o [B][Nq][D], k, v [B][Nk][D] (dtype f16 or bf16, contiguous).
 * Follows the FlashAttention test's arithmetic
 * (test/python/triton/test_flash_attention.py, attention_fwd_kernel /
 * _attn_fwd_inner): qk = sum_d q*k in binary32 (d ascending),
 * t = qk * (scale * log2 e), m = max_j t, p = exp2(t - m), l = sum_j p,
 * O = (sum_j p * v) / l.  The reference folds the blocks online; a single
 * block holding the whole row is the same recurrence with alpha = 1.
 * causal: key j is visible to query i iff j <= i. */
void hxo_attention(const void* q, const void* k, const void* v, void* o, int dtype,
                   int64_t B, int64_t Nq, int64_t Nk, int64_t D, float scale, int causal)
{
    const float qk_scale = scale * 1.44269504088896340736f;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b) {
        for (int64_t i = 0; i < Nq; ++i) {
            float t[16384];  /* Nk <= 16384 (checked by the wrapper) */
            const int64_t qo = (b * Nq + i) * D;
            float m = -INFINITY;
            for (int64_t j = 0; j < Nk; ++j) {
                if (causal && j > i) { t[j] = -INFINITY; continue; }
                const int64_t ko = (b * Nk + j) * D;
                float acc = 0.0f;
                for (int64_t d = 0; d < D; ++d)
                    acc += load_elem(q, dtype, qo + d) * load_elem(k, dtype, ko + d);
                t[j] = acc * qk_scale;
                if (t[j] > m) m = t[j];
            }
            float l = 0.0f;
            for (int64_t j = 0; j < Nk; ++j) {
                t[j] = (t[j] == -INFINITY) ? 0.0f : exp2f(t[j] - m);
                l += t[j];
            }
            for (int64_t d = 0; d < D; ++d) {
                float acc = 0.0f;
                for (int64_t j = 0; j < Nk; ++j)
                    acc += t[j] * load_elem(v, dtype, (b * Nk + j) * D + d);
                store_elem(o, dtype, qo + d, l > 0.0f ? acc / l : 0.0f);
            }
        }
    }
}
