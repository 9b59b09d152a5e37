// hx_probe.hip -- measurement probes for bench.py's --ceilings mode (built
// into libhxprobe.so, not part of the hx ABI).  They measure what this box
// sustains, as the denominators the kernels' rooflines are read against:
//   * the period of back-to-back launches of an empty kernel (the launch
//     gap every short kernel pays when timed back to back);
//   * a streaming read and a copy of a given size (16-byte non-temporal
//     loads, grid-stride), the HBM ceiling of the GEMV and the row ops;
//   * v_mfma_i32_32x32x32_i8 issued back to back on register operands (the
//     MFMA ceiling at the clock the chip holds under that load), alone and
//     with the LDS operand reads of the GEMM's 128x64 wave tile beside it.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__global__ void probe_empty_kernel() {}

// Streaming read: XOR of every 16-byte word; one word per block reaches
// memory only if the XOR hits a magic value (it never does for the fills
// used), so the loads cannot be dropped.
__global__ void __launch_bounds__(256) probe_read_kernel(const v4i* __restrict__ p, int64_t n16, int* sink) {
  v4i acc = v4i{0, 0, 0, 0};
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    acc ^= __builtin_nontemporal_load(p + i);
  const int x = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (x == 0x5eed1234) sink[blockIdx.x] = x;
}

__global__ void __launch_bounds__(256) probe_copy_kernel(const v4i* __restrict__ s, v4i* __restrict__ d,
                                                         int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    __builtin_nontemporal_store(__builtin_nontemporal_load(s + i), d + i);
}

// The same copy in the one-row-per-workgroup pattern of the row kernels:
// workgroup b copies the 8 KiB at 8192 b with two 16-byte loads per thread
// (both issued before either store), as a softmax row of 4096 fp16 is read
// and written.
__global__ void __launch_bounds__(256) probe_copy_rows_kernel(const v4i* __restrict__ s, v4i* __restrict__ d,
                                                              int64_t n16) {
  const int64_t base = (int64_t)blockIdx.x * 512;
  v4i v[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    if (i < n16) v[u] = __builtin_nontemporal_load(s + i);
  }
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int64_t i = base + u * 256 + threadIdx.x;
    if (i < n16) __builtin_nontemporal_store(v[u], d + i);
  }
}

// 8 independent int8 MFMA chains per wave, `iters` rounds of 8 MFMAs; NR
// 16-byte LDS reads per round beside them (6 is the GEMM's 128x64 wave
// tile), and NG coalesced 16-byte-per-lane loads of an L2-resident 1 MiB
// buffer (operands that bypass LDS).  The reads' results feed the next
// round's operands, so they cannot be dropped; LDS lanes read 16 bytes at an
// 80-byte stride (conflict-free).
template <int NR, int NG>
__global__ void __launch_bounds__(512) probe_mfma_kernel(int iters, const v4i* __restrict__ g, int* out) {
  __shared__ v4i tile[NR ? 4096 : 1];
  const int lane = threadIdx.x & 63;
  v4i a[2], b[4];
  for (int i = 0; i < 2; ++i) a[i] = v4i{lane + i, 1, 2, 3};
  for (int j = 0; j < 4; ++j) b[j] = v4i{j, lane, 5, 7};
  if constexpr (NR > 0) {
    for (int i = threadIdx.x; i < 4096; i += 512) tile[i] = v4i{i, i + 1, i + 2, i + 3};
    __syncthreads();
  }
  v16i acc[8];
  for (int t = 0; t < 8; ++t) acc[t] = v16i{};
  const int base = (threadIdx.x * 5) & 4095;
  const int gw = (int)(blockIdx.x * 8 + (threadIdx.x >> 6)) * 97;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[4 * i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[4 * i + j], 0, 0, 0);
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const v4i t = tile[(base + 64 * r + it) & 4095];
      if (r % 6 < 2) a[r % 6] ^= t;
      else b[r % 6 - 2] ^= t;
    }
#pragma unroll
    for (int q = 0; q < NG; ++q) {
      const v4i t = g[((gw + it * NG + q) * 64 + lane) & 65535];
      b[(q + 2) & 3] ^= t;
    }
  }
  int s = 0;
  for (int t = 0; t < 8; ++t)
    for (int r = 0; r < 16; ++r) s += acc[t][r];
  if (s == 0x5eed1234) out[blockIdx.x] = s;
}

// One wave per SIMD (4 per CU) with a 128x128 wave tile: 16 independent
// MFMA chains (256 accumulator registers), `iters` rounds of 16 MFMAs with NR
// LDS reads per round (8 is the tile's operand traffic: 4 A + 4 B).  The
// operands are double-buffered as a GEMM would hold them: a round's reads
// land in the other register set and feed the round after the next one.
template <int NR>
__global__ void __launch_bounds__(256) probe_mfma4_kernel(int iters, int* out) {
  __shared__ v4i tile[4096];
  const int lane = threadIdx.x & 63;
  v4i a[2][4], b[2][4];
  for (int s = 0; s < 2; ++s) {
    for (int i = 0; i < 4; ++i) a[s][i] = v4i{lane + i + s, 1, 2, 3};
    for (int j = 0; j < 4; ++j) b[s][j] = v4i{j + s, lane, 5, 7};
  }
  for (int i = threadIdx.x; i < 4096; i += 256) tile[i] = v4i{i, i + 1, i + 2, i + 3};
  __syncthreads();
  v16i acc[16];
  for (int t = 0; t < 16; ++t) acc[t] = v16i{};
  const int base = (threadIdx.x * 5) & 4095;
  for (int it = 0; it < iters; it += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      // reads for the other set, spread between this set's MFMAs
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[4 * i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][i], b[s][j], acc[4 * i + j], 0, 0, 0);
          const int r = 4 * i + j;
          if (r < NR) {
            const v4i t = tile[(base + 64 * r + it + s) & 4095];
            if (r < 4) a[s ^ 1][r] ^= t;
            else b[s ^ 1][r - 4] ^= t;
          }
        }
    }
  }
  int s = 0;
  for (int t = 0; t < 16; ++t)
    for (int r = 0; r < 16; ++r) s += acc[t][r];
  if (s == 0x5eed1234) out[blockIdx.x] = s;
}

// Two schedules of the same work: 8 waves, 8 int8 MFMA chains each, 6
// 16-byte LDS operand reads per 8 MFMAs (the GEMM's 128x64 wave tile), the
// operands of R rounds of 8 MFMAs read ahead.
// Ping-pong: waves 0-3 and 4-7 (one of each per SIMD) alternate an MFMA
// burst of R rounds with the read burst for their next one, workgroup
// barriers between the phases and the second group one phase behind
// (PRIO: the MFMA burst at raised wave priority).  Every wave passes the
// same number of barriers.
template <int R, int PRIO>
__global__ void __launch_bounds__(512) probe_pingpong_kernel(int phases, int* out) {
  __shared__ v4i tile[4096];
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 4096; i += 512) tile[i] = v4i{i, i + 1, i + 2, i + 3};
  __syncthreads();
  const int grp = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 8));
  v4i a[R][2], b[R][4];
  for (int r = 0; r < R; ++r) {
    for (int i = 0; i < 2; ++i) a[r][i] = v4i{lane + i + r, 1, 2, 3};
    for (int j = 0; j < 4; ++j) b[r][j] = v4i{j + r, lane, 5, 7};
  }
  v16i acc[8];
  for (int t = 0; t < 8; ++t) acc[t] = v16i{};
  const int base = (threadIdx.x * 5) & 4095;
  if (grp == 1) __builtin_amdgcn_s_barrier();
  for (int ph = 0; ph < phases; ++ph) {
    // memory phase: the next compute phase's operands
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int q = 0; q < 6; ++q) {
        const v4i t = tile[(base + 64 * (6 * r + q) + ph) & 4095];
        if (q < 2) a[r][q] ^= t;
        else b[r][q - 2] ^= t;
      }
    __builtin_amdgcn_s_barrier();
    if (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[4 * i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[r][i], b[r][j], acc[4 * i + j], 0, 0, 0);
    if (PRIO) __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_s_barrier();
  }
  if (grp == 0) __builtin_amdgcn_s_barrier();
  int s = 0;
  for (int t = 0; t < 8; ++t)
    for (int r = 0; r < 16; ++r) s += acc[t][r];
  if (s == 0x5eed1234) out[blockIdx.x] = s;
}

// Interleaved: every wave spreads the reads of its next R rounds between
// the MFMAs of these (the GEMM kernel's schedule), no group barriers.
template <int R>
__global__ void __launch_bounds__(512) probe_interleave_kernel(int phases, int* out) {
  __shared__ v4i tile[4096];
  const int lane = threadIdx.x & 63;
  for (int i = threadIdx.x; i < 4096; i += 512) tile[i] = v4i{i, i + 1, i + 2, i + 3};
  __syncthreads();
  v4i a[2][R][2], b[2][R][4];
  for (int s = 0; s < 2; ++s)
    for (int r = 0; r < R; ++r) {
      for (int i = 0; i < 2; ++i) a[s][r][i] = v4i{lane + i + r + s, 1, 2, 3};
      for (int j = 0; j < 4; ++j) b[s][r][j] = v4i{j + r + s, lane, 5, 7};
    }
  v16i acc[8];
  for (int t = 0; t < 8; ++t) acc[t] = v16i{};
  const int base = (threadIdx.x * 5) & 4095;
  for (int ph = 0; ph < phases; ph += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            acc[4 * i + j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s][r][i], b[s][r][j], acc[4 * i + j], 0, 0, 0);
            const int q = 4 * i + j;
            if (q < 6) {
              const v4i t = tile[(base + 64 * (6 * r + q) + ph + s) & 4095];
              if (q < 2) a[s ^ 1][r][q] ^= t;
              else b[s ^ 1][r][q - 2] ^= t;
            }
          }
  }
  int s = 0;
  for (int t = 0; t < 8; ++t)
    for (int r = 0; r < 16; ++r) s += acc[t][r];
  if (s == 0x5eed1234) out[blockIdx.x] = s;
}


// A read of the decode GEMV's weight in a GEMV launch shape (N = 11008,
// K = 4096 int8, the packed image: 688 tiles of 64 chunks of 1 KiB; CT tiles
// per workgroup of KW waves, wave w loading chunks w + KW u of each tile with
// 16-byte buffer loads), with the column-scale load first and the LDS
// exchange and barrier at the end, and no arithmetic: what the GEMV's memory
// side alone costs in that shape.  CT = 3, KW = 16 is the default's shape
// (230 workgroups).  The data is folded into one word per lane so no load is
// dead.
template <int CT, int KW>
__global__ void __launch_bounds__(64 * KW) probe_read_tiles_kernel(const char* __restrict__ p, long bytes,
                                                                  const float* sc, int nsc, int* sink) {
  constexpr int CPW = 64 / KW;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const long region = (long)CT * 64 * 1024;
  const long rem = bytes - (long)blockIdx.x * region;
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p + (long)blockIdx.x * region), 0, rem < region ? (int)rem : (int)region, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)sc, 0, nsc * 4, 0x00020000);
  const unsigned s0 =
      __builtin_amdgcn_raw_buffer_load_b32(rs, (int)((blockIdx.x * 16 * CT + (tid % (16 * CT))) * 4), 0, 0);
  v4i v[CPW * CT];
#pragma unroll
  for (int u = 0; u < CPW; ++u)
#pragma unroll
    for (int c = 0; c < CT; ++c)
      v[u * CT + c] = __builtin_bit_cast(
          v4i, __builtin_amdgcn_raw_buffer_load_b128(rw, (c * 64 + wave + KW * u) * 1024 + lane * 16, 0, 2));
  v4i acc{0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < CPW * CT; ++j) acc ^= v[j];
  __shared__ unsigned red[KW][64];
  red[wave][lane] = (unsigned)(acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) ^ s0;
  __syncthreads();
  if (tid < 64) {
    unsigned q = 0;
    for (int w = 0; w < KW; ++w) q ^= red[w][tid];
    if (q == 0x5eed1234u) sink[1] = 1;
  }
}
extern "C" {
// blocks x 512 threads: the schedules above (kind 0, 1: interleaved, 1 or 2
// rounds read ahead; 2..6: ping-pong with R = 1, 1, 2, 2, 4 rounds per
// phase, the odd kinds and 6 with raised priority); `phases` phases of R
// rounds; int8 ops per launch in *ops
int hxp_mfma_sched_i8(int kind, int blocks, int phases, int* out, double* ops, hipStream_t s) {
  int r = 0;
  switch (kind) {
    case 0: probe_interleave_kernel<1><<<blocks, 512, 0, s>>>(phases, out); r = 1; break;
    case 1: probe_interleave_kernel<2><<<blocks, 512, 0, s>>>(phases, out); r = 2; break;
    case 2: probe_pingpong_kernel<1, 0><<<blocks, 512, 0, s>>>(phases, out); r = 1; break;
    case 3: probe_pingpong_kernel<1, 1><<<blocks, 512, 0, s>>>(phases, out); r = 1; break;
    case 4: probe_pingpong_kernel<2, 0><<<blocks, 512, 0, s>>>(phases, out); r = 2; break;
    case 5: probe_pingpong_kernel<2, 1><<<blocks, 512, 0, s>>>(phases, out); r = 2; break;
    case 6: probe_pingpong_kernel<4, 1><<<blocks, 512, 0, s>>>(phases, out); r = 4; break;
    default: return -1;
  }
  *ops = (double)blocks * 8 /*waves*/ * phases * r * 8 /*mfma*/ * 65536.0;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// blocks x 256 threads (4 waves, 128x128 wave tiles), 0, 4 or 8 LDS reads
// per 16 MFMAs
int hxp_mfma4_i8(int blocks, int iters, int lds_reads, int* out, double* ops, hipStream_t s) {
  if (lds_reads == 0) probe_mfma4_kernel<0><<<blocks, 256, 0, s>>>(iters, out);
  else if (lds_reads == 4) probe_mfma4_kernel<4><<<blocks, 256, 0, s>>>(iters, out);
  else if (lds_reads == 8) probe_mfma4_kernel<8><<<blocks, 256, 0, s>>>(iters, out);
  else return -1;
  *ops = (double)blocks * 4 /*waves*/ * iters * 16 /*mfma*/ * 65536.0;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

// one launch of probe_read_tiles_kernel<CT, KW> over `bytes` (whole 64 KiB
// tiles; the last workgroup's range is cut to the buffer), column scales
// `sc` [nsc] binary32; (CT, KW) in {(3, 16), (3, 8), (1, 8), (1, 4)}
int hxp_read_tiles(int ct, int kw, const void* p, int64_t bytes, const float* sc, int nsc, int* sink,
                   hipStream_t s) {
  const char* q = (const char*)p;
  const long tiles = (long)((bytes + 65535) / 65536);
  const unsigned g = (unsigned)((tiles + ct - 1) / ct);
  if (ct == 3 && kw == 16) probe_read_tiles_kernel<3, 16><<<g, 1024, 0, s>>>(q, bytes, sc, nsc, sink);
  else if (ct == 3 && kw == 8) probe_read_tiles_kernel<3, 8><<<g, 512, 0, s>>>(q, bytes, sc, nsc, sink);
  else if (ct == 1 && kw == 8) probe_read_tiles_kernel<1, 8><<<g, 512, 0, s>>>(q, bytes, sc, nsc, sink);
  else if (ct == 1 && kw == 4) probe_read_tiles_kernel<1, 4><<<g, 256, 0, s>>>(q, bytes, sc, nsc, sink);
  else return -1;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
// the default's shape (three tiles over 16 waves)
int hxp_read_gemv_shape(const void* p, int64_t bytes, const float* sc, int nsc, int* sink, hipStream_t s) {
  return hxp_read_tiles(3, 16, p, bytes, sc, nsc, sink, s);
}
int hxp_empty(hipStream_t s) {
  probe_empty_kernel<<<1, 64, 0, s>>>();
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int hxp_read(const void* p, int64_t bytes, int blocks, int* sink, hipStream_t s) {
  probe_read_kernel<<<blocks, 256, 0, s>>>((const v4i*)p, bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
// one workgroup per 8 KiB
int hxp_copy_rows(const void* src, void* dst, int64_t bytes, hipStream_t s) {
  const int64_t n16 = bytes / 16;
  probe_copy_rows_kernel<<<(unsigned)((n16 + 511) / 512), 256, 0, s>>>((const v4i*)src, (v4i*)dst, n16);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
int hxp_copy(const void* src, void* dst, int64_t bytes, int blocks, hipStream_t s) {
  probe_copy_kernel<<<blocks, 256, 0, s>>>((const v4i*)src, (v4i*)dst, bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : -1;
}
// blocks x 512 threads (8 waves): `lds_reads` LDS reads and `global_loads`
// buffer loads (of `g`, 1 MiB) per 8 MFMAs, for the combinations below;
// returns int8 ops per launch in *ops
int hxp_mfma_i8(int blocks, int iters, int lds_reads, int global_loads, const void* g, int* out, double* ops,
                hipStream_t s) {
  const v4i* gv = (const v4i*)g;
#define HXP_CASE(R, G)                                                            \
  if (lds_reads == R && global_loads == G) {                                      \
    probe_mfma_kernel<R, G><<<blocks, 512, 0, s>>>(iters, gv, out);               \
    *ops = (double)blocks * 8 /*waves*/ * iters * 8 /*mfma*/ * 65536.0;           \
    return hipGetLastError() == hipSuccess ? 0 : -1;                              \
  }
  HXP_CASE(0, 0) HXP_CASE(2, 0) HXP_CASE(4, 0) HXP_CASE(6, 0)
  HXP_CASE(0, 2) HXP_CASE(0, 4) HXP_CASE(0, 6) HXP_CASE(4, 2) HXP_CASE(2, 4)
#undef HXP_CASE
  return -1;
}
}
