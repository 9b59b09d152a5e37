// hx_device.hpp -- device-side building blocks shared by the hx kernels
// (gfx950 / CDNA4 only): vector types, exact narrowing conversions, 64-lane
// wave reductions and thin wrappers over the MFMA builtins.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace hx {

// Compile-time loop: f(std::integral_constant<int, I>) for I = 0..N-1, as a
// fold expression, so indices into register arrays are constants no matter
// how large the body is (an unroller threshold cannot demote the array to
// scratch memory).
template <class F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

typedef _Float16 f16;
typedef uint16_t bf16_bits;  // bf16 is carried as raw bits and converted by hand

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

enum DType : int { DT_F16 = 1, DT_BF16 = 2, DT_F32 = 3, DT_I8 = 4, DT_I32 = 5 };

// ---------------------------------------------------------------------------
// Scalar conversions.  fp32 -> fp16 uses v_cvt_f16_f32 (round to nearest
// even in the default mode); fp32 -> bf16 is written out so that the rounding
// (RNE, quiet NaN) is explicit and identical to the CPU oracle.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t x = __float_as_uint(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  // The empty asm makes f an opaque binary32 value: without it the backend
  // folds a preceding multiply into the conversion (v_fma_mixlo_f16, one
  // rounding instead of two) even with floating-point contraction off.
  asm("" : "+v"(f));
  f16 h = (f16)f;
  return __builtin_bit_cast(uint16_t, h);
}
// Two binary32 values -> packed fp16 pair (low = a), each rounded to nearest
// even: one v_cvt_pk_f16_f32.  The asm keeps a and b opaque for the same
// reason as in f32_to_f16_bits.
__device__ __forceinline__ uint32_t f32x2_to_f16x2(float a, float b) {
  asm("" : "+v"(a), "+v"(b));
  typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, hf2{(f16)a, (f16)b});
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(f16, h);
}

// Element access for the three floating storage types used by row kernels.
template <int DT> struct Elem;
template <> struct Elem<DT_F16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(storage v) { return f16_bits_to_f32(v); }
  static __device__ __forceinline__ storage store(float v) { return f32_to_f16_bits(v); }
};
template <> struct Elem<DT_BF16> {
  typedef uint16_t storage;
  static __device__ __forceinline__ float load(storage v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ storage store(float v) { return f32_to_bf16(v); }
};
template <> struct Elem<DT_F32> {
  typedef float storage;
  static __device__ __forceinline__ float load(storage v) { return v; }
  static __device__ __forceinline__ storage store(float v) { return v; }
};

// ---------------------------------------------------------------------------
// Wave-wide (64-lane) reductions.  DPP row shifts / swizzles are selected by
// the compiler from __shfl_xor; every lane ends up with the full result.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// exp(x) = 2^(x*log2(e)) on the hardware v_exp_f32 (1 ulp on exp2).  The
// argument here is always <= 0 (softmax after max subtraction) or bounded
// (SiLU), so the prescale's relative error stays at the 1e-7 level.
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// The SwiGLU gate on fp16 values: RNE(silu(g) * u), silu(g) = g / (1 +
// exp(-g)) in binary32 (correctly rounded divide); shared by the silu_mul
// kernel and the decode GEMV's fused epilogue so both give the same bits.
__device__ __forceinline__ uint16_t silu_mul_h(uint16_t g, uint16_t u) {
  const float x = f16_bits_to_f32(g);
  const float sx = x / (1.0f + fast_exp(-x));
  return f32_to_f16_bits(sx * f16_bits_to_f32(u));
}

// ---------------------------------------------------------------------------
// int8 -> fp16 conversion of four packed signed bytes into two half2 words.
// (b ^ 0x80) is the byte as an unsigned excess-128 value u in [1, 255]; the
// half with bits 0x6400 | u is 1024 + u exactly, so subtracting 1152 gives
// the signed value exactly.  Two v_perm_b32 + one packed f16 subtract.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void i8x4_to_f16x4(uint32_t w, v2h& lo, v2h& hi) {
  const uint32_t u = w ^ 0x80808080u;
  // v_perm_b32(src0, src1, sel): byte k of the result = byte sel_k of the
  // 8-byte value {src0:src1} (src1 supplies bytes 0-3, src0 bytes 4-7).
  const uint32_t lo_bits = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
  const uint32_t hi_bits = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
  const v2h bias = {(f16)1152.0f, (f16)1152.0f};
  lo = __builtin_bit_cast(v2h, lo_bits) - bias;
  hi = __builtin_bit_cast(v2h, hi_bits) - bias;
}

// Eight int8 values (two dwords) -> one MFMA f16 operand (8 halves).
__device__ __forceinline__ v8h i8x8_to_v8h(uint32_t w0, uint32_t w1) {
  v2h a, b, c, d;
  i8x4_to_f16x4(w0, a, b);
  i8x4_to_f16x4(w1, c, d);
  v8h r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// The same conversion for bytes already stored in excess-128 form
// (u = b ^ 0x80, as the packed decode-GEMV weight image keeps them): the
// XOR is done once when the image is built instead of on every load.
__device__ __forceinline__ v8h x8x8_to_v8h(uint32_t u0, uint32_t u1) {
  const v2h bias = {(f16)1152.0f, (f16)1152.0f};
  v8h r;
  const v2h a = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) - bias;
  const v2h b = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) - bias;
  const v2h c = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) - bias;
  const v2h d = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) - bias;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// ---------------------------------------------------------------------------
// MFMA wrappers.  All 32x32 variants take a 16-byte A and B operand per lane:
// lane l supplies row (l % 32) and the 16-byte K slice (l / 32), and the 16
// accumulator registers of lane l hold column (l % 32), rows
// 8*(r/4) + 4*(l/32) + (r%4).
// ---------------------------------------------------------------------------
__device__ __forceinline__ v16i mfma32_i8(v4i a, v4i b, v16i c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma32_f16(v4i a, v4i b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a),
                                                 __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}
__device__ __forceinline__ v16f mfma32_bf16(v4i a, v4i b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a),
                                                  __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}
// 16x16x32 f16: lane l supplies row (l % 16), K slice 8*(l/16)..+7; the four
// accumulator registers of lane l hold column (l % 16), rows 4*(l/16) + r.
__device__ __forceinline__ v4f mfma16_f16(v8h a, v8h b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Cache policy of buffer stores whose lines should not wait dirty in L2 for
// the end-of-kernel write-back: SC0 | SC1 (system-scope coherent, i.e.
// written through to memory).
constexpr int kStoreWriteThrough = 1 | 16;
// SC1 alone: the cache policy of an agent-scope atomic access on gfx942 /
// gfx950 (stores written through the XCD's L2, loads not served by a stale
// line of it).  Used for data one workgroup hands to another through memory.
constexpr int kAgentCoherent = 16;

// ---- direct-to-LDS staging (GEMM and attention) -------------------------
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

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding):
// all but this wave's N most recent direct-to-LDS loads have landed.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that orders LDS only.  __syncthreads() is a release
// fence on all memory, which counts outstanding direct-to-LDS loads as
// pending LDS writes and forces vmcnt(0); here every wave has already waited
// for its own loads of the stage it is about to publish (wait_vm), so the
// barrier needs only this wave's LDS reads retired (lgkmcnt(0)).  The
// "memory" clobber keeps the compiler from moving memory operations across
// it, the sched_barriers keep the machine scheduler from doing so.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}


}  // namespace hx
