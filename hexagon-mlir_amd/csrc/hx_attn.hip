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
// rows); each wave owns 32 query rows.  K/V blocks of 64 or 128 keys are staged
// through LDS, double-buffered, with the next block's global loads in flight
// during the current block's MFMAs.  Scores are computed transposed
// (S^T = K . Q^T with v_mfma_f32_32x32x16_{f16,bf16}) so that every lane
// holds one query row and 16 of its keys: row max and row sum are in-lane
// plus one exchange with the partner lane (lane ^ 32), and the exponentials
// are already in the operand layout of the P . V product -- no cross-lane
// shuffle of P.  V is stored transposed in LDS (keys contiguous) so that the
// P . V operand of a lane is two 8-byte reads.
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

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  if constexpr (DT == DT_BF16) return (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
  else return (uint32_t)f32_to_f16_bits(a) | ((uint32_t)f32_to_f16_bits(b) << 16);
}

// 16-byte chunk swizzles.  K rows are D*2 bytes (D/8 chunks): the 32 rows an
// operand read touches land on distinct bank groups.  V^T rows are BN*2
// bytes: for 128-byte rows (64 keys) (d>>1 ^ d>>3), for 256-byte rows
// (128 keys) (d ^ d>>3), keep both the transposing 2-byte writes (rows 8
// apart) and the 8-byte operand reads (16 consecutive rows) conflict-free.
template <int D>
__device__ __forceinline__ int swz_k(int row) {
  if constexpr (D == 64) return (row ^ (row >> 3)) & 7;
  else return row & 15;
}
template <int BN>
__device__ __forceinline__ int swz_vt(int d) {
  if constexpr (BN == 64) return ((d >> 1) ^ (d >> 3)) & 7;
  else return (d ^ (d >> 3)) & 15;
}

}  // namespace

template <int D, int DT, bool CAUSAL, int ATT_BN>
__global__ void __launch_bounds__(256) attn_fwd_kernel(AttnArgs p) {
  constexpr int KS = D / 16;             // MFMA k-steps of the score product
  constexpr int DTILES = D / 32;         // 32-wide output column tiles
  constexpr int JT = ATT_BN / 32;        // 32-key score tiles per block
  constexpr int PS = ATT_BN / 16;        // 16-key steps of the P . V product
  constexpr int VROW = ATT_BN * 2;       // bytes per V^T row
  constexpr int K_BYTES = ATT_BN * D * 2;
  constexpr int VT_BYTES = D * ATT_BN * 2;
  constexpr int CPR = D / 8;             // 16-byte chunks per K/V row
  constexpr int LOADS = ATT_BN * CPR / 256;  // 16-byte chunks per thread per block (each of K and V)
  static_assert(LOADS >= 1 && ATT_BN * CPR % 256 == 0, "block split");
  __shared__ __attribute__((aligned(16))) char sk[2][K_BYTES];
  __shared__ __attribute__((aligned(16))) char svt[2][VT_BYTES];

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
  const float qk_scale = p.scale * 1.44269504088896340736f;

  // Key blocks this workgroup visits (causal: up to its last query row).
  int64_t nk = p.Nk;
  if constexpr (CAUSAL) {
    const int64_t last_q = min((int64_t)qb * ATT_BM + ATT_BM, p.Nq) - 1 + p.causal_offset;
    nk = min(nk, last_q + 1);
  }
  const int nblk = nk > 0 ? (int)((nk + ATT_BN - 1) / ATT_BN) : 0;

  // Global -> registers for one K/V block: thread chunk u = tid + 256*r is
  // row u / CPR (key), 16-byte column chunk u % CPR.  Buffer loads: rows
  // past Nk fall outside the descriptor's range and read as zero, with no
  // branch.
  const uint32_t k_bytes = (uint32_t)(((p.Nk - 1) * p.sk[2] + D) * 2);
  const uint32_t v_bytes = (uint32_t)(((p.Nk - 1) * p.sv[2] + D) * 2);
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc((void*)k, 0, (int)k_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc((void*)v, 0, (int)v_bytes, 0x00020000);
  v4i kr[LOADS], vr[LOADS];
  auto load_block = [&](int blk) {
    static_for<LOADS>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      const int u = tid + 256 * r;
      const int64_t key = (int64_t)blk * ATT_BN + u / CPR;
      const int c = u % CPR;
      const bool in = key < p.Nk;
      const uint32_t ko = in ? (uint32_t)((key * p.sk[2] + 8 * c) * 2) : 0x80000000u;
      const uint32_t vo = in ? (uint32_t)((key * p.sv[2] + 8 * c) * 2) : 0x80000000u;
      kr[r] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rk, (int)ko, 0, 0));
      vr[r] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rv, (int)vo, 0, 0));
    });
  };
  // Registers -> LDS buffer b: K row-major (swizzled chunks), V transposed.
  auto store_block = [&](int b) {
    static_for<LOADS>([&](auto rc) {
      constexpr int r = decltype(rc)::value;
      const int u = tid + 256 * r;
      const int key = u / CPR, c = u % CPR;
      *reinterpret_cast<v4i*>(&sk[b][key * D * 2 + ((c ^ swz_k<D>(key)) << 4)]) = kr[r];
      const uint32_t w[4] = {(uint32_t)vr[r][0], (uint32_t)vr[r][1], (uint32_t)vr[r][2],
                             (uint32_t)vr[r][3]};
      static_for<8>([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        const int d = 8 * c + i;
        const uint16_t h = (uint16_t)(w[i >> 1] >> (16 * (i & 1)));
        *reinterpret_cast<uint16_t*>(
            &svt[b][d * VROW + (((key >> 3) ^ swz_vt<ATT_BN>(d)) << 4) + (key & 7) * 2]) = h;
      });
    });
  };

  if (nblk > 0) {
    load_block(0);
    store_block(0);
  }
  __syncthreads();

  for (int blk = 0; blk < nblk; ++blk) {
    const int b = blk & 1;
    if (blk + 1 < nblk) load_block(blk + 1);  // in flight during this block

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
        kf[ks] = *reinterpret_cast<const v4i*>(&sk[b][krow * D * 2 + ((c ^ swz_k<D>(krow)) << 4)]);
      });
      __builtin_amdgcn_sched_barrier(0);
      s[jt] = v16f{};
      static_for<KS>([&](auto kc) {
        constexpr int ks = decltype(kc)::value;
        s[jt] = mfma_att<DT>(kf[ks], qf[ks], s[jt]);
      });
    });
    __builtin_amdgcn_sched_barrier(0);

    // mask, row max, online-softmax update (exp2 domain, as the reference)
    const int64_t key0 = (int64_t)blk * ATT_BN;
    float mx = -INFINITY;
    // Only a block that reaches past Nk, or (causal) past the workgroup's
    // first query row, needs the per-element mask.
    bool full = key0 + ATT_BN <= p.Nk;
    if constexpr (CAUSAL) full = full && key0 + ATT_BN - 1 <= (int64_t)qb * ATT_BM + p.causal_offset;
    if (full) {
      static_for<JT>([&](auto jc) {
        constexpr int jt = decltype(jc)::value;
        static_for<16>([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          const float t = s[jt][r] * qk_scale;
          s[jt][r] = t;
          mx = fmaxf(mx, t);
        });
      });
    } else {
      static_for<JT>([&](auto jc) {
        constexpr int jt = decltype(jc)::value;
        static_for<16>([&](auto rc) {
          constexpr int r = decltype(rc)::value;
          const int64_t key = key0 + 32 * jt + 8 * (r >> 2) + 4 * lg + (r & 3);
          bool keep = key < p.Nk;
          if constexpr (CAUSAL) keep = keep && key <= q_row + p.causal_offset;
          const float t = keep ? s[jt][r] * qk_scale : -INFINITY;
          s[jt][r] = t;
          mx = fmaxf(mx, t);
        });
      });
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_i, mx);
    // a row with every key masked so far keeps m = -inf; exponentiate
    // against 0 then so that p = 0 and alpha = 1 instead of NaN
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_fast(m_i - m_use);
    float rs = 0.f;
    static_for<JT>([&](auto jc) {
      constexpr int jt = decltype(jc)::value;
      static_for<16>([&](auto rc) {
        constexpr int r = decltype(rc)::value;
        const float e = exp2_fast(s[jt][r] - m_use);
        s[jt][r] = e;
        rs += e;
      });
    });
    rs += __shfl_xor(rs, 32);
    l_i = l_i * alpha + rs;
    m_i = m_new;
    static_for<DTILES>([&](auto dc) {
      constexpr int dt = decltype(dc)::value;
      static_for<16>([&](auto rc) { oacc[dt][decltype(rc)::value] *= alpha; });
    });

    // O^T += V^T . P^T over the block's 16-key steps.  Step t covers keys
    // 16t + 4*lg + (0..3) and 16t + 8 + 4*lg + (0..3) in this lane's k slots:
    // exactly the exponentials held in score registers 4g..4g+3, g = 2t' and
    // 2t'+1 (t' = t % 2) of tile t/2 -- and the matching V^T reads.
    v4i pf[PS];
    static_for<PS>([&](auto tc) {
      constexpr int t = decltype(tc)::value;
      constexpr int jt = t >> 1, g0 = 2 * (t & 1);
      pf[t] = v4i{(int)pack2<DT>(s[jt][4 * g0 + 0], s[jt][4 * g0 + 1]),
                  (int)pack2<DT>(s[jt][4 * g0 + 2], s[jt][4 * g0 + 3]),
                  (int)pack2<DT>(s[jt][4 * g0 + 4], s[jt][4 * g0 + 5]),
                  (int)pack2<DT>(s[jt][4 * g0 + 6], s[jt][4 * g0 + 7])};
    });
    static_for<DTILES>([&](auto dc) {
      constexpr int dt = decltype(dc)::value;
      const int d = 32 * dt + lrow;
      const char* row = &svt[b][d * VROW];
      v4i vf[PS];
      static_for<PS>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        const int ka = 16 * t + 4 * lg, kb = ka + 8;
        const v2i lo = *reinterpret_cast<const v2i*>(row + (((ka >> 3) ^ swz_vt<ATT_BN>(d)) << 4) + (ka & 7) * 2);
        const v2i hi = *reinterpret_cast<const v2i*>(row + (((kb >> 3) ^ swz_vt<ATT_BN>(d)) << 4) + (kb & 7) * 2);
        vf[t] = v4i{lo[0], lo[1], hi[0], hi[1]};
      });
      static_for<PS>([&](auto tc) {
        constexpr int t = decltype(tc)::value;
        oacc[dt] = mfma_att<DT>(vf[t], pf[t], oacc[dt]);
      });
    });

    if (blk + 1 < nblk) {
      store_block(b ^ 1);
    }
    __syncthreads();
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

template <int D, int DT, bool CAUSAL, int BN>
static void attn_launch(const AttnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.Nq + ATT_BM - 1) / ATT_BM), (unsigned)(a.Z * a.H));
  attn_fwd_kernel<D, DT, CAUSAL, BN><<<grid, dim3(256), 0, s>>>(a);
}

const char* attn_refusal(const AttnArgs& a) {
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  if (a.D != 64 && a.D != 128) return "head-dim";
  if (!al16(a.q) || !al16(a.k) || !al16(a.v) || !al16(a.o)) return "unaligned-base";
  for (int i = 0; i < 3; ++i)
    if (a.sq[i] % 8 || a.sk[i] % 8 || a.sv[i] % 8 || a.so[i] % 8) return "row-stride";
  if (a.Z * a.H > 65535 || (a.Nq + ATT_BM - 1) / ATT_BM > 0x7fffffff) return "grid";
  return nullptr;
}

int launch_attention(int dtype, bool causal, const AttnArgs& a, hipStream_t s) {
  if (attn_refusal(a)) return HXI_ERR_UNSUPPORTED;
  if (a.Nq == 0 || a.Z * a.H == 0) return HXI_OK;
  // keys per K/V block: 64 for D = 64 (two workgroups fit a CU), 128 for
  // D = 128 (half the per-block softmax bookkeeping)
#define HX_ATT(D_, DT_, BN_)                                     \
  if (a.D == D_ && dtype == DT_) {                               \
    if (causal) attn_launch<D_, DT_, true, BN_>(a, s);           \
    else attn_launch<D_, DT_, false, BN_>(a, s);                 \
    return HXI_OK;                                               \
  }
  HX_ATT(64, DT_F16, 64)
  HX_ATT(128, DT_F16, 128)
  HX_ATT(64, DT_BF16, 64)
  HX_ATT(128, DT_BF16, 128)
#undef HX_ATT
  return HXI_ERR_UNSUPPORTED;
}

}  // namespace hx
