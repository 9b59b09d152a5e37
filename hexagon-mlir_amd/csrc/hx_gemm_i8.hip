// hx_gemm_i8.hip -- the int8 x int8 config table of the MFMA GEMM family
// (kernel template in hx_gemm_kernel.hpp, dispatch in hx_gemm.hip).
#include "hx_gemm_kernel.hpp"

namespace hx {

// A host function holding the table: a namespace-scope array of host
// function pointers would also be emitted by the device compilation.
const GemmEntry* gemm_table_i8(int& n) {
  static const GemmEntry t[] = {
      HX_GEMM_CFGS(GM_I8),
      // K stage width and depth: 64-byte stages halve the LDS per stage
      // (room for a third stage, or more workgroups per CU), 256-byte stages
      // halve the barriers per K
      {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_bk64", 1, 0.86f, 0, 64, 2},
       &launch_one<GM_I8, 256, 256, 2, 4, GE_STORE, 64, 2>},
      {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_bk64_s3", 1, 0.92f, 0, 64, 3},
       &launch_one<GM_I8, 256, 256, 2, 4, GE_STORE, 64, 3>},
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_bk64", 2, 0.71f, 0, 64, 2},
       &launch_one<GM_I8, 128, 128, 2, 2, GE_STORE, 64, 2>},
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_bk64_s3", 2, 0.68f, 0, 64, 3},
       &launch_one<GM_I8, 128, 128, 2, 2, GE_STORE, 64, 3>},
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_bk256", 1, 0.67f, 0, 256, 2},
       &launch_one<GM_I8, 128, 128, 2, 2, GE_STORE, 256, 2>},
      {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_bk256", 2, 0.51f, 0, 256, 2},
       &launch_one<GM_I8, 64, 64, 2, 2, GE_STORE, 256, 2>},
      // persistent (one workgroup per CU walking consecutive M-tiles of a B
      // strip, each tile's epilogue overlapping the next tile's first K
      // stages): 64-byte stages leave LDS room for the epilogue's own
      // staging region
      {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_bk64_p", 1, 0.80f, 0, 64, 2, 1},
       &launch_one<GM_I8, 256, 256, 2, 4, GE_STORE, 64, 2, 1, true>},
      {{128, 256, 2, 4, GE_STORE, "128x256_w2x4_p", 1, 0.75f, 0, 128, 2, 1},
       &launch_one<GM_I8, 128, 256, 2, 4, GE_STORE, 128, 2, 1, true>},
      // K in parts (int32 partials, exact, and a merge that dequantises):
      // fills the chip when the output tiles are fewer than the CUs
      {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_k2", 1, 1.00f, 2}, &launch_one<GM_I8, 256, 256, 2, 4, GE_STORE, 128, 2, 1, false, true>},
      {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_k2", 2, 0.89f, 2}, &launch_one<GM_I8, 128, 128, 2, 2, GE_STORE, 128, 2, 1, false, true>},
      {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_k4", 4, 0.61f, 4}, &launch_one<GM_I8, 64, 64, 2, 2, GE_STORE, 128, 2, 1, false, true>},
      // a deeper split of the same kernel for skinny products with a long K
      // (f16 512x512x8192: 17.0 against 20.9 us in four parts; 16 parts
      // measured slower than 8 everywhere)
      {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_k8", 4, 0.61f, 8}, &launch_one<GM_I8, 64, 64, 2, 2, GE_STORE, 128, 2, 1, false, true>},
  };
  n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace hx
