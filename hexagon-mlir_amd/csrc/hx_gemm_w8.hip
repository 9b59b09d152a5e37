// hx_gemm_w8.hip -- the f16 x int8 (W8A16, incl. SwiGLU) config table of the MFMA GEMM family
// (kernel template in hx_gemm_kernel.hpp, dispatch in hx_gemm.hip).
#include "hx_gemm_kernel.hpp"

namespace hx {

// A host function holding the table: a namespace-scope array of host
// function pointers would also be emitted by the device compilation.
const GemmEntry* gemm_table_w8(int& n) {
  static const GemmEntry t[] = {
    HX_GEMM_CFGS(GM_W8),
    {{256, 128, 2, 4, GE_SWIGLU, "swiglu_256x128_w2x4", 1, 0.95f}, &launch_one<GM_W8, 256, 128, 2, 4, GE_SWIGLU>},
    {{256, 128, 2, 2, GE_SWIGLU, "swiglu_256x128_w2x2", 1, 0.77f}, &launch_one<GM_W8, 256, 128, 2, 2, GE_SWIGLU>},
    {{128, 128, 2, 2, GE_SWIGLU, "swiglu_128x128_w2x2", 1, 0.80f}, &launch_one<GM_W8, 128, 128, 2, 2, GE_SWIGLU>},
    {{128, 64, 2, 2, GE_SWIGLU, "swiglu_128x64_w2x2", 2, 0.80f}, &launch_one<GM_W8, 128, 64, 2, 2, GE_SWIGLU>},
    // persistent: one workgroup per CU walks consecutive M-tiles of one
    // weight strip (the SwiGLU gate/up block's 688 tiles at 2048 x 11008 are
    // 2.7 tiles per CU), each tile's epilogue overlapping the next tile's
    // first K stages
    {{256, 128, 2, 4, GE_SWIGLU, "swiglu_256x128_w2x4_p", 1, 0.90f, 0, 128, 2, 1},
     &launch_one<GM_W8, 256, 128, 2, 4, GE_SWIGLU, 128, 2, 1, true>},
    {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_p", 1, 0.95f, 0, 128, 2, 1},
     &launch_one<GM_W8, 256, 256, 2, 4, GE_STORE, 128, 2, 1, true>},
    // K in two parts (binary32 partials and a merge): the FFN down
    // projection's 2048x4096 output is 128 tiles of 256x256 for 256 CUs
    {{256, 256, 2, 4, GE_STORE, "256x256_w2x4_k2", 1, 1.00f, 2}, &launch_one<GM_W8, 256, 256, 2, 4, GE_STORE, 128, 2, 1, false, true>},
    // the same output as 256 tiles of half the width, eight waves of 64x64
    // each: the chip is full without a K split, so no partials and no merge
    {{256, 128, 4, 2, GE_STORE, "256x128_w4x2", 1, 0.90f}, &launch_one<GM_W8, 256, 128, 4, 2, GE_STORE>},
    {{128, 256, 2, 4, GE_STORE, "128x256_w2x4", 1, 0.90f}, &launch_one<GM_W8, 128, 256, 2, 4, GE_STORE>},
    // small tiles with K in parts: more workgroups per CU for skinny M
    {{128, 128, 2, 2, GE_STORE, "128x128_w2x2_k2", 2, 0.89f, 2}, &launch_one<GM_W8, 128, 128, 2, 2, GE_STORE, 128, 2, 1, false, true>},
    {{64, 64, 2, 2, GE_STORE, "64x64_w2x2_k4", 4, 0.61f, 4}, &launch_one<GM_W8, 64, 64, 2, 2, GE_STORE, 128, 2, 1, false, true>},
};
  n = (int)(sizeof(t) / sizeof(t[0]));
  return t;
}

}  // namespace hx
