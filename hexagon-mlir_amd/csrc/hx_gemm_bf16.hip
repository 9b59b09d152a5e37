// hx_gemm_bf16.hip -- the bf16 x bf16 config table of the MFMA GEMM family
// (kernel template in hx_gemm_kernel.hpp, dispatch in hx_gemm.hip).
#include "hx_gemm_kernel.hpp"

namespace hx {

// A host function holding the table: a namespace-scope array of host
// function pointers would also be emitted by the device compilation.
const GemmEntry* gemm_table_bf16(int& n) {
  static const GemmEntry t[] = {
      HX_GEMM_CFGS(GM_BF16),
      // K in two parts (binary32 partials and a merge): fills the chip when
      // the 256x256 tiles of a long-K product are fewer than the CUs
      {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_k2", 1, 1.00f, 2}, &launch_one<GM_BF16, 256, 256, 2, 4, GE_STORE, 128, 2, 1, false, true>},
      // small tiles with K in parts: more workgroups per CU for skinny M
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_k2", 2, 0.89f, 2}, &launch_one<GM_BF16, 128, 128, 2, 2, GE_STORE, 128, 2, 1, false, true>},
      {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_k4", 4, 0.61f, 4}, &launch_one<GM_BF16, 64, 64, 2, 2, GE_STORE, 128, 2, 1, false, true>},
      // a deeper split of the same kernel for skinny products with a long K
      // (f16 512x512x8192: 17.0 against 20.9 us in four parts; 16 parts
      // measured slower than 8 everywhere)
      {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_k8", 4, 0.61f, 8}, &launch_one<GM_BF16, 64, 64, 2, 2, GE_STORE, 128, 2, 1, false, true>},
      // K stage width and depth (a 128-byte stage is 64 k): 256-byte stages
      // halve the barriers per K of a deep product; three 64-byte stages
      // keep two stages of loads in flight
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_bk256", 1, 0.67f, 0, 256, 2},
       &launch_one<GM_BF16, 128, 128, 2, 2, GE_STORE, 256, 2>},
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_bk64_s3", 2, 0.68f, 0, 64, 3},
       &launch_one<GM_BF16, 128, 128, 2, 2, GE_STORE, 64, 3>},
  };
  n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace hx
