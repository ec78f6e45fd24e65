// Implicit-GEMM convolution instantiations (NDHWC activation, DHWIO weights, NDHWC output):
// M = N*OD*OH*OW output pixels, N = O output channels, K = KD*KH*KW*C.
//   *_fast_*_d  C % 64 == 0: each 64-wide K-tile is one filter tap; direct-to-LDS gather (padding
//               taps read as zero), weights staged [K][O] and read transposed
//   *_gen_*_vV  any C: register-staged gather with per-group tap decode, V-wide loads
#include "tile_direct.hpp"

using namespace mtk;

// 256x256 tiles: 8 wavefronts (2 x 4, two per SIMD, one workgroup per CU); 128x128: 4 (2 x 2, two
// workgroups per CU).
#define DIRECT_KERNEL(NAME, BM, BN, WM, WN)                                                          \
  extern "C" __global__ void __launch_bounds__(64 * WM * WN) NAME(const mtk_tile_args a) {        \
    tile_direct<DT_F16, BM, BN, WM, WN, OpConv<BM, WM * WN>, OpColsT<BN, WM * WN>>(a);            \
  }

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

DIRECT_KERNEL(mtk_conv_f16_fast_256x256_d, 256, 256, 2, 4)
DIRECT_KERNEL(mtk_conv_f16_fast_128x128_d, 128, 128, 2, 2)

TILE_KERNEL(mtk_conv_f16_gen_128x128_v8, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 8, 8)
TILE_KERNEL(mtk_conv_f16_gen_128x128_v4, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 4, 4)
TILE_KERNEL(mtk_conv_f16_gen_128x128_v1, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 1, 1)
