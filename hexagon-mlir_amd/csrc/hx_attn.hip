// hx_attn.hip -- fused scaled-dot-product attention forward for gfx950:
//   O = softmax(Q K^T * scale [causal mask]) V,  binary32 scores and
//   accumulation, exp2-based online softmax, fp16/bf16 in and out.
//
// What it replaces in hexagon-mlir: the FlashAttention composition its
// Triton front end lowers (test/python/triton/test_flash_attention.py:
// _attn_fwd_inner and attention_fwd_kernel) -- per K/V block of BLOCK_N keys:
// qk = q . k^T; m_ij = max(m_i, rowmax(qk) * qk_scale); p = exp2(qk * qk_scale
// - m_ij); l_i = l_i * exp2(m_i - m_ij) + rowsum(p); acc = acc * alpha +
// p . v; finally O = acc / l_i, with qk_scale = sm_scale * log2(e) -- and the
// online-softmax recurrence of test/python/triton/test_online_softmax.py.
//
// MI355X design: one workgroup of four waves per (batch*head, 128 query
// rows); each wave owns 32 query rows.  K/V blocks of 64 or 128 keys are
// staged row-major in LDS by direct-to-LDS buffer loads (no register
// staging), double-buffered: the next block's loads are in flight during the
// current block's MFMAs.  Scores are computed transposed (S^T = K . Q^T with
// v_mfma_f32_32x32x16_{f16,bf16}) so that every lane holds one query row and
// 16 of its keys: row max and row sum are in-lane plus one exchange with the
// partner lane (lane ^ 32), and the exponentials are already in the operand
// layout of the P . V product -- no cross-lane shuffle of P.  The V^T
// operand of P . V is read from the row-major V block with gfx950's
// transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group,
// lane 4a+b receives element b of the 8-byte chunks addressed by lanes
// a, a+4, a+8, a+12, i.e. one column of V across four consecutive keys.
#include "hx_device.hpp"
#include "hx_internal.hpp"

namespace hx {

namespace {

constexpr int ATT_BM = 128;  // query rows per workgroup

template <int DT>
__device__ __forceinline__ v16f mfma_att(v4i a, v4i b, v16f c) {
  if constexpr (DT == DT_BF16) return mfma32_bf16(a, b, c);
  else return mfma32_f16(a, b, c);
}

// 2^x on the transcendental unit (v_exp_f32), without the library's
// denormal-result rescaling: a probability below 2^-126 contributes nothing
// at binary32 accumulation precision anyway.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// two binary32 values rounded to nearest-even and packed (v_cvt_pk_f16_f32 /
// v_cvt_pk_bf16_f32: one instruction per pair)
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == DT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, bf2{(__bf16)a, (__bf16)b});
  } else {
    typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, hf2{(_Float16)a, (_Float16)b});
  }
}

// Lazy rescaling: the running row maximum m is only moved (and the output
// accumulator rescaled) when a block's maximum exceeds it by more than
// RESCALE_MARGIN (log2 units); otherwise the block's probabilities are
// exponentiated against the old m and may reach 2^RESCALE_MARGIN, which
// fp16/bf16 P and the binary32 sums hold without loss (the final O = acc / l
// is independent of which m was used).
constexpr float RESCALE_MARGIN = 8.0f;

// 16-byte chunk swizzles of the row-major K and V blocks (rows of D*2
// bytes, D/8 chunks).  K: the 32 rows a score-operand read touches land on
// distinct bank groups.  V: the transposing reads of a half wave cover 4
// consecutive keys x 32 bytes (D = 64: 8 keys over two 128-byte rows per
// bank period); XOR-ing the chunk with 4*(row & 3) (D = 128) or
// 4*((row >> 1) & 1) (D = 64) spreads them over all 64 banks.  The direct
// loads write whole KiB runs, conflict-free under any swizzle.
template <int D>
__device__ __forceinline__ int swz_k(int row) {
  if constexpr (D == 64) return (row ^ (row >> 3)) & 7;
  else return row & 15;
}
template <int D>
__device__ __forceinline__ int swz_v(int row) {
  if constexpr (D == 64) return 4 * ((row >> 1) & 1);
  else return 4 * (row & 3);
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v4s* lds_v4s_ptr;

}  // namespace

// SPLIT: the workgroup covers key-block range `blockIdx.z` of `p.splits`
// equal ranges of its query block's blocks, and instead of O it writes the
// unnormalised binary32 accumulator with its row maximum m (exp2 domain) and
// row sum l to `p.part`; attn_combine_kernel merges the ranges.  Partial
// layout, for partial row r = (bh * splits + split) * Nq + query:
//   acc at part[r * D + d], (m, l) at part[R * D + 2 * r + {0, 1}],
//   R = Z * H * splits * Nq.
template <int D, int DT, bool CAUSAL, int ATT_BN, bool SPLIT>
__global__ void __launch_bounds__(256) attn_fwd_kernel(AttnArgs p) {
  constexpr int KS = D / 16;             // MFMA k-steps of the score product
  constexpr int DTILES = D / 32;         // 32-wide output column tiles
  constexpr int JT = ATT_BN / 32;        // 32-key score tiles per block
  constexpr int PS = ATT_BN / 16;        // 16-key steps of the P . V product
  constexpr int ROWB = D * 2;            // bytes per K or V row
  constexpr int CPR = D / 8;             // 16-byte chunks per row
  constexpr int RPK = 1024 / ROWB;       // rows per 1 KiB direct load
  constexpr int BLK_BYTES = ATT_BN * ROWB;
  constexpr int PER_W = BLK_BYTES / 4096;  // direct loads per wave per operand per block
  static_assert(PER_W >= 1 && BLK_BYTES % 4096 == 0, "block split");
  static_assert(2 * PER_W < 64, "vmcnt range");
  // two buffers as distinct arrays, so the compiler can see that a direct
  // load into one never aliases the reads of the other
  __shared__ __attribute__((aligned(1024))) char sk0[BLK_BYTES];
  __shared__ __attribute__((aligned(1024))) char sv0[BLK_BYTES];
  __shared__ __attribute__((aligned(1024))) char sk1[BLK_BYTES];
  __shared__ __attribute__((aligned(1024))) char sv1[BLK_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lrow = lane & 31, lg = lane >> 5;
  // Workgroup -> (head, query block): heads vary fastest over consecutive
  // workgroup ids (which the dispatcher deals to the 8 XCDs in turn), query
  // blocks are taken last-first, so under a causal mask the long rows start
  // first and every XCD gets the same mix of long and short rows.
  const int nbh = (int)(p.Z * p.H);
  const int lin = blockIdx.x + gridDim.x * blockIdx.y;
  const int bh = __builtin_amdgcn_readfirstlane(lin % nbh);
  const int qb = __builtin_amdgcn_readfirstlane((int)gridDim.x - 1 - lin / nbh);
  const int zb = bh / (int)p.H, hb = bh - zb * (int)p.H;
  const char* q = reinterpret_cast<const char*>(p.q) + 2 * (zb * p.sq[0] + hb * p.sq[1]);
  const char* k = reinterpret_cast<const char*>(p.k) + 2 * (zb * p.sk[0] + hb * p.sk[1]);
  const char* v = reinterpret_cast<const char*>(p.v) + 2 * (zb * p.sv[0] + hb * p.sv[1]);
  char* o = reinterpret_cast<char*>(p.o) + 2 * (zb * p.so[0] + hb * p.so[1]);
  const int64_t q_row = (int64_t)qb * ATT_BM + wave * 32 + lrow;  // this lane's query
  const bool q_in = q_row < p.Nq;

  // Q operand fragments: row q_row, d = 16*ks + 8*lg + (0..7)
  v4i qf[KS];
  static_for<KS>([&](auto kc) {
    constexpr int ks = decltype(kc)::value;
    qf[ks] = q_in ? *reinterpret_cast<const v4i*>(q + 2 * (q_row * p.sq[2] + 16 * ks + 8 * lg))
                  : v4i{0, 0, 0, 0};
  });

  v16f oacc[DTILES];
  static_for<DTILES>([&](auto dc) { oacc[decltype(dc)::value] = v16f{}; });
  float m_i = -INFINITY, l_i = 0.f;
  // exp2-domain scale; exponent arguments are fma(s, qk_scale, -m).  A
  // negative scale is moved into Q (an exact sign flip of every element, so
  // S flips sign exactly); a zero scale becomes a tiny positive one, which
  // leaves every finite score at 2^0 and keeps masked (-inf) scores at 0.
  float qk_scale = p.scale * 1.44269504088896340736f;
  if (qk_scale < 0.f) {
    static_for<KS>([&](auto kc) { qf[decltype(kc)::value] ^= (int)0x80008000u; });
    qk_scale = -qk_scale;
  }
  qk_scale = fmaxf(qk_scale, 1e-30f);

  // Key blocks this workgroup visits (causal: up to its last query row).
  int64_t nk = p.Nk;
  if constexpr (CAUSAL) {
    const int64_t last_q = min((int64_t)qb * ATT_BM + ATT_BM, p.Nq) - 1 + p.causal_offset;
    nk = min(nk, last_q + 1);
  }
  const int nblk_all = nk > 0 ? (int)((nk + ATT_BN - 1) / ATT_BN) : 0;
  // this workgroup's key blocks [b0, b0 + nblk)
  int b0 = 0, nblk = nblk_all;
  if constexpr (SPLIT) {
    const int per = (nblk_all + p.splits - 1) / p.splits;
    b0 = min((int)blockIdx.z * per, nblk_all);
    nblk = min(per, nblk_all - b0);
  }

  // Direct loads of key block blk: load i of wave w fills the KiB of rows
  // (w + 4i)*RPK + lane/CPR; the lane writes physical chunk lane % CPR and
  // fetches the logical chunk the row's swizzle maps there.  Rows past Nk
  // get an offset outside the buffer descriptor's range and read as zero.
  const uint32_t sk_b = (uint32_t)(p.sk[2] * 2), sv_b = (uint32_t)(p.sv[2] * 2);
  const uint32_t k_bytes = (uint32_t)(((p.Nk - 1) * p.sk[2] + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((p.Nk - 1) * p.sv[2] + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, (int)k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, (int)v_bytes, 0x00020000);
  // The lane's part of each offset (its row within the block and swizzled
  // chunk) is fixed; the block's first key enters as the uniform scalar
  // offset.  Only a block that reaches past Nk selects per row.
  uint32_t k_lane[PER_W], v_lane[PER_W];
  int row_l[PER_W];
  static_for<PER_W>([&](auto ic) {
    constexpr int i = decltype(ic)::value;
    const int row = (wave + 4 * i) * RPK + lane / CPR, pc = lane % CPR;
    row_l[i] = row;
    k_lane[i] = (uint32_t)row * sk_b + (uint32_t)((pc ^ swz_k<D>(row)) << 4);
    v_lane[i] = (uint32_t)row * sv_b + (uint32_t)((pc ^ swz_v<D>(row)) << 4);
  });
  auto dma_block = [&](char* dk, char* dv, int blk) {
    const int64_t key0 = (int64_t)blk * ATT_BN;
    const uint32_t ks = (uint32_t)key0 * sk_b, vs = (uint32_t)key0 * sv_b;
    if (key0 + ATT_BN <= p.Nk) {
      static_for<PER_W>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        dma16(rk, dk + (wave + 4 * i) * 1024, k_lane[i], ks);
        dma16(rv, dv + (wave + 4 * i) * 1024, v_lane[i], vs);
      });
    } else {
      const int lim = (int)(p.Nk - key0);
      static_for<PER_W>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const bool in = row_l[i] < lim;
        dma16(rk, dk + (wave + 4 * i) * 1024, in ? k_lane[i] : 0x80000000u, ks);
        dma16(rv, dv + (wave + 4 * i) * 1024, in ? v_lane[i] : 0x80000000u, vs);
      });
    }
  };

  // The V^T operand of 16-key step t, keys 16t + 8*half + 4*lg + (0..3) of
  // column d = 32*dt + lrow: lane 16G + a + 4j addresses key
  // 16t + 8*half + 4*(G/2) + j, columns 32*dt + 16*(G%2) + 4a + (0..3).
  auto read_vt = [&](const char* cv, int dt, int t, int half) -> v2i {
    const int row = 16 * t + 8 * half + 4 * (lane >> 5) + ((lane & 15) >> 2);
    const int col = 32 * dt + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    const char* a = cv + row * ROWB + (((col >> 3) ^ swz_v<D>(row)) << 4) + ((col >> 2) & 1) * 8;
    return __builtin_bit_cast(v2i, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_ptr)a));
  };

  auto block = [&](const char* ck, const char* cv, int blk) {
    // S^T = K . Q^T: lane holds query q_row, keys 32*jt + 8*g + 4*lg + (0..3).
    // Per 32-key tile, its K fragment reads are issued before its MFMAs.
    v16f s[JT];
    static_for<JT>([&](auto jc) {
      constexpr int jt = decltype(jc)::value;
      const int krow = 32 * jt + lrow;
      v4i kf[KS];
      static_for<KS>([&](auto kc) {
        constexpr int ks = decltype(kc)::value;
        const int c = 2 * ks + lg;
        kf[ks] = *reinterpret_cast<const v4i*>(ck + krow * ROWB + ((c ^ swz_k<D>(krow)) << 4));
      });
      __builtin_amdgcn_sched_barrier(0);
      s[jt] = mfma_att<DT>(kf[0], qf[0], v16f{});
      static_for<KS - 1>([&](auto kc) {
        constexpr int ks = decltype(kc)::value + 1;
        s[jt] = mfma_att<DT>(kf[ks], qf[ks], s[jt]);
      });
    });
    __builtin_amdgcn_sched_barrier(0);

    // mask, row max, online-softmax update (exp2 domain, as the reference)
    const int64_t key0 = (int64_t)blk * ATT_BN;
    float mx = -INFINITY;
    // Only a block that reaches past Nk, or (causal) past the workgroup's
    // first query row, needs the per-element mask: keys key0 + rel with
    // rel >= lim are masked to -inf.
    bool full = key0 + ATT_BN <= p.Nk;
    if constexpr (CAUSAL) full = full && key0 + ATT_BN - 1 <= (int64_t)qb * ATT_BM + p.causal_offset;
    if (full) {
      static_for<JT>([&](auto jc) {
        constexpr int jt = decltype(jc)::value;
        static_for<16>([&](auto rc) { mx = fmaxf(mx, s[jt][decltype(rc)::value]); });
      });
    } else {
      int64_t lim64 = min((int64_t)ATT_BN, p.Nk - key0);
      if constexpr (CAUSAL) lim64 = min(lim64, q_row + p.causal_offset - key0 + 1);
      // this lane's keys are rel = c + 4*lg for compile-time c: compare c
      // against lim - 4*lg (no per-element index registers)
      const int lim_l = (int)max(lim64, (int64_t)0) - 4 * lg;
      static_for<JT>([&](auto jc) {
        constexpr int jt = decltype(jc)::value;
        static_for<16>([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          constexpr int c = 32 * jt + 8 * (r >> 2) + (r & 3);
          const float t = c < lim_l ? s[jt][r] : -INFINITY;
          s[jt][r] = t;
          mx = fmaxf(mx, t);
        });
      });
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mxs = mx == -INFINITY ? -INFINITY : mx * qk_scale;
    const bool grow = mxs > m_i + RESCALE_MARGIN;  // -inf + margin stays -inf
    if (__builtin_amdgcn_ballot_w64(grow)) {
      const float m_new = grow ? mxs : m_i;
      const float alpha = grow ? exp2_fast(m_i - m_new) : 1.f;
      l_i *= alpha;
      m_i = m_new;
      static_for<DTILES>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        static_for<16>([&](auto rc) { oacc[dt][decltype(rc)::value] *= alpha; });
      });
    }
    // a row with every key masked so far keeps m = -inf; exponentiate
    // against 0 then so that p = 0 instead of NaN
    const float mu = m_i == -INFINITY ? 0.f : m_i;
    // O^T += V^T . P^T, one 16-key step at a time: step t covers keys
    // 16t + 4*lg + (0..3) and 16t + 8 + 4*lg + (0..3) in this lane's k
    // slots -- exactly the scores held in registers 4g..4g+3, g = 2t' and
    // 2t'+1 (t' = t % 2) of tile t/2.  The step's exponentials are taken,
    // packed and multiplied into every column tile before the next step's
    // are taken, so they run under the previous step's MFMAs; each column
    // tile still accumulates the steps in order, and the row sum adds the
    // exponentials in the same order as one pass over the block would.
    // D = 128: each step, from its V^T reads to its MFMAs, runs at wave
    // priority 1 (s_setprio), so the SIMD issues it ahead of the other
    // wave's instructions and the step's MFMAs reach the matrix core sooner
    // (MI355X, interleaved A/B: causal 4096 x 2048 x 128 heads 5% faster,
    // non-causal 1-2%; D = 64 7% slower with it, so it stays at 0 there).
    float rs = 0.f;
    static_for<PS>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      constexpr int jt = t >> 1, g0 = 2 * (t & 1);
      if constexpr (D == 128) __builtin_amdgcn_s_setprio(1);
      v4i vf[DTILES];
      static_for<DTILES>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        const v2i lo = read_vt(cv, dt, t, 0);
        const v2i hi = read_vt(cv, dt, t, 1);
        vf[dt] = v4i{lo[0], lo[1], hi[0], hi[1]};
      });
      float e[8];
      static_for<8>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        e[r] = exp2_fast(__builtin_fmaf(s[jt][4 * g0 + r], qk_scale, -mu));
        rs += e[r];
      });
      const v4i pf = v4i{(int)pack2<DT>(e[0], e[1]), (int)pack2<DT>(e[2], e[3]), (int)pack2<DT>(e[4], e[5]),
                         (int)pack2<DT>(e[6], e[7])};
      static_for<DTILES>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        oacc[dt] = mfma_att<DT>(vf[dt], pf, oacc[dt]);
      });
      if constexpr (D == 128) __builtin_amdgcn_s_setprio(0);
    });
    rs += __shfl_xor(rs, 32);
    l_i += rs;
  };

  // Blocks in pairs over the two buffers; each block's loads were issued
  // one block earlier and are published by the barrier that ends it.
  if (nblk > 0) dma_block(sk0, sv0, b0);
  wait_vm<0>();
  lds_barrier();
  int i = 0;
  for (; i + 2 <= nblk; i += 2) {
    dma_block(sk1, sv1, b0 + i + 1);
    block(sk0, sv0, b0 + i);
    wait_vm<0>();
    lds_barrier();
    if (i + 2 < nblk) dma_block(sk0, sv0, b0 + i + 2);
    block(sk1, sv1, b0 + i + 1);
    wait_vm<0>();
    lds_barrier();
  }
  if (i < nblk) block(sk0, sv0, b0 + i);

  if constexpr (SPLIT) {
    // lane holds accumulator columns 32*dt + 8*g + 4*lg + (0..3) of its row;
    // both lanes of a row hold the same m and l
    if (q_in) {
      const int64_t r = ((int64_t)bh * p.splits + blockIdx.z) * p.Nq + q_row;
      float* po = p.part + r * D;
      static_for<DTILES>([&](auto dc) {
        constexpr int dt = decltype(dc)::value;
        static_for<4>([&](auto gc) {
          constexpr int g = decltype(gc)::value;
          *reinterpret_cast<v4f*>(po + 32 * dt + 8 * g + 4 * lg) =
              v4f{oacc[dt][4 * g], oacc[dt][4 * g + 1], oacc[dt][4 * g + 2], oacc[dt][4 * g + 3]};
        });
      });
      if (lg == 0) {
        const int64_t R = p.Z * p.H * p.splits * p.Nq;
        *reinterpret_cast<v2f*>(p.part + R * D + 2 * r) = v2f{m_i, l_i};
      }
    }
    return;
  }

  // O = acc / l: lane holds row q_row, columns 32*dt + 8*g + 4*lg + (0..3)
  if (q_in) {
    const float inv = l_i > 0.f ? 1.0f / l_i : 0.f;
    static_for<DTILES>([&](auto dc) {
      constexpr int dt = decltype(dc)::value;
      static_for<4>([&](auto gc) {
        constexpr int g = decltype(gc)::value;
        const int d = 32 * dt + 8 * g + 4 * lg;
        const v2i w = v2i{(int)pack2<DT>(oacc[dt][4 * g] * inv, oacc[dt][4 * g + 1] * inv),
                          (int)pack2<DT>(oacc[dt][4 * g + 2] * inv, oacc[dt][4 * g + 3] * inv)};
        *reinterpret_cast<v2i*>(o + 2 * (q_row * p.so[2] + d)) = w;
      });
    });
  }
}

// Merge of the key-range partials of attn_fwd_kernel<..., SPLIT = true>:
// with M = max_s m_s and w_s = 2^(m_s - M),
//   O = (sum_s w_s acc_s) / (sum_s w_s l_s),
// the online-softmax recurrence applied once across the ranges.  A range
// that saw only masked keys has m = -inf, l = 0, acc = 0 and weight 0; a
// row with no visible key at all gets O = 0, as in the single pass.  Each
// thread finalises four consecutive columns of one query row.  The loop
// over ranges is unrolled to SMAX with the range index clamped to the last
// one (its weight then forced to 0), so every partial load of the thread is
// issued before the first is used: one round trip to memory, not one per
// range.
template <int D, int DT, int SMAX>
__global__ void __launch_bounds__(256) attn_combine_kernel(AttnArgs p) {
  constexpr int TPR = D / 4;  // threads per row
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t rows = p.Z * p.H * p.Nq;
  if (t >= rows * TPR) return;
  const int64_t row = t / TPR;  // bh * Nq + query
  const int d = 4 * (int)(t - row * TPR);
  const int64_t bh = row / p.Nq, qr = row - bh * p.Nq;
  const int S = p.splits;
  const float* ml = p.part + rows * S * D;
  const int64_t r0 = bh * S * p.Nq + qr;  // partial row of range 0; range s adds s * Nq
  v2f mls[SMAX];
  v4f accs[SMAX];
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    const int64_t r = r0 + (int64_t)min(s, S - 1) * p.Nq;
    mls[s] = *reinterpret_cast<const v2f*>(ml + 2 * r);
    accs[s] = *reinterpret_cast<const v4f*>(p.part + r * D + d);
  }
  float M = -INFINITY;
#pragma unroll
  for (int s = 0; s < SMAX; ++s) M = fmaxf(M, mls[s][0]);  // clamped copies repeat a real range
  float L = 0.f;
  v4f acc = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < SMAX; ++s) {
    const float w = (s < S && mls[s][0] != -INFINITY) ? exp2_fast(mls[s][0] - M) : 0.f;
    L += w * mls[s][1];
    acc += w * accs[s];
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const int64_t zb = bh / p.H, hb = bh - zb * p.H;
  char* o = reinterpret_cast<char*>(p.o) + 2 * (zb * p.so[0] + hb * p.so[1] + qr * p.so[2] + d);
  *reinterpret_cast<v2i*>(o) = v2i{(int)pack2<DT>(acc[0] * inv, acc[1] * inv),
                                   (int)pack2<DT>(acc[2] * inv, acc[3] * inv)};
}

// Split the key range when the (head, query block) workgroups would fill
// less than half of the 256 CUs: enough ranges to bring the grid to about
// 256 workgroups, each at least kMinSplitBlocks key blocks long, at most
// kMaxSplits ranges.  Measured at Z = H = 1, N = 1024, D = 64: 8 ranges
// 9.0 us, 16 ranges 9.7 us, 4 ranges 10.8 us, single pass 15.7 us.
constexpr int kMinSplitBlocks = 2;
constexpr int kMaxSplits = 8;

template <int D, int DT, bool CAUSAL, int BN>
static void attn_launch(const AttnArgs& a, hipStream_t s) {
  const unsigned qblocks = (unsigned)((a.Nq + ATT_BM - 1) / ATT_BM);
  if (a.splits > 1) {
    const dim3 grid(qblocks, (unsigned)(a.Z * a.H), (unsigned)a.splits);
    attn_fwd_kernel<D, DT, CAUSAL, BN, true><<<grid, dim3(256), 0, s>>>(a);
    const int64_t threads = a.Z * a.H * a.Nq * (D / 4);
    const dim3 cgrid((unsigned)((threads + 255) / 256));
    // the combine's unrolled range count: the smallest of 2, 4, 8 that holds
    // every range (each unused slot costs a load per thread)
    if (a.splits <= 2) attn_combine_kernel<D, DT, 2><<<cgrid, dim3(256), 0, s>>>(a);
    else if (a.splits <= 4) attn_combine_kernel<D, DT, 4><<<cgrid, dim3(256), 0, s>>>(a);
    else attn_combine_kernel<D, DT, kMaxSplits><<<cgrid, dim3(256), 0, s>>>(a);
  } else {
    attn_fwd_kernel<D, DT, CAUSAL, BN, false><<<dim3(qblocks, (unsigned)(a.Z * a.H)), dim3(256), 0, s>>>(a);
  }
}

// Keys per block of the launched kernels (see launch_attention).
constexpr int ATT_BN_ALL = 64;
int attn_splits(const AttnArgs& a) {
  const int64_t wgs = (a.Nq + ATT_BM - 1) / ATT_BM * a.Z * a.H;
  const int64_t nblk = (a.Nk + ATT_BN_ALL - 1) / ATT_BN_ALL;
  if (wgs <= 0 || wgs >= 128 || nblk < 2 * kMinSplitBlocks) return 1;
  int64_t sp = (256 + wgs - 1) / wgs;
  sp = std::min<int64_t>(sp, nblk / kMinSplitBlocks);
  sp = std::min<int64_t>(sp, kMaxSplits);
  return (int)std::max<int64_t>(sp, 1);
}
size_t attn_part_bytes(const AttnArgs& a) {
  if (a.splits <= 1) return 0;
  return (size_t)(a.Z * a.H * a.Nq) * (size_t)a.splits * (size_t)(a.D + 2) * sizeof(float);
}

const char* attn_refusal(const AttnArgs& a) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.D != 64 && a.D != 128) return "head-dim";
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || !al16(a.o)) return "unaligned-base";
  for (int i = 0; i < 3; ++i)
    if (a.sq[i] % 8 || a.sk[i] % 8 || a.sv[i] % 8 || a.so[i] % 8) return "row-stride";
  if (a.Z * a.H > 65535 || (a.Nq + ATT_BM - 1) / ATT_BM > 0x7fffffff) return "grid";
  // K and V rows of one head are addressed with 32-bit byte offsets
  if (a.Nk > 0 && (((a.Nk - 1) * a.sk[2] + a.D) * 2 >= ((int64_t)1 << 31) ||
                   ((a.Nk - 1) * a.sv[2] + a.D) * 2 >= ((int64_t)1 << 31)))
    return "offset-range";
  return nullptr;
}

int launch_attention(int dtype, bool causal, const AttnArgs& a, hipStream_t s) {
  if (attn_refusal(a)) return HXI_ERR_UNSUPPORTED;
  if (a.Nq == 0 || a.Z * a.H == 0) return HXI_OK;
  if (a.splits > 1 && (a.part == nullptr || a.splits > kMaxSplits)) return HXI_ERR_ARG;
  // keys per K/V block: 64 (MI355X sweep over 32 / 64 / 128 keys; with
  // 64 keys a D = 128 workgroup needs 64 KiB of LDS, two fit a CU)
#define HX_ATT(D_, DT_, BN_)                                     \
  if (a.D == D_ && dtype == DT_) {                               \
    if (causal) attn_launch<D_, DT_, true, BN_>(a, s);           \
    else attn_launch<D_, DT_, false, BN_>(a, s);                 \
    return HXI_OK;                                               \
  }
  static_assert(ATT_BN_ALL == 64, "attn_splits counts 64-key blocks");
  static_assert(kMaxSplits == 8, "attn_launch instantiates the combine for 2, 4 and 8 ranges");
  HX_ATT(64, DT_F16, 64)
  HX_ATT(128, DT_F16, 64)
  HX_ATT(64, DT_BF16, 64)
  HX_ATT(128, DT_BF16, 64)
#undef HX_ATT
  return HXI_ERR_UNSUPPORTED;
}

}  // namespace hx
