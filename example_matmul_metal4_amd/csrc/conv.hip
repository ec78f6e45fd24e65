// Implicit-GEMM convolution instantiations (NDHWC activation, DHWIO weights, NDHWC output):
// M = N*OD*OH*OW output pixels, N = O output channels, K = KD*KH*KW*C. "fast" kernels need
// C % 64 == 0 (each 64-wide K-tile lies in one filter tap); "gen" kernels take any C.
#include "tile_gemm.hpp"

using namespace mtk;

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

TILE_KERNEL(mtk_conv_f16_fast_256x256_v8, DT_F16, 256, 256, 2, 2, A_CONV, B_KN, 8, 8)
TILE_KERNEL(mtk_conv_f16_fast_256x256_v4, DT_F16, 256, 256, 2, 2, A_CONV, B_KN, 8, 4)
TILE_KERNEL(mtk_conv_f16_fast_256x256_v1, DT_F16, 256, 256, 2, 2, A_CONV, B_KN, 8, 1)
TILE_KERNEL(mtk_conv_f16_fast_256x128_v8, DT_F16, 256, 128, 2, 2, A_CONV, B_KN, 8, 8)
TILE_KERNEL(mtk_conv_f16_fast_256x128_v4, DT_F16, 256, 128, 2, 2, A_CONV, B_KN, 8, 4)
TILE_KERNEL(mtk_conv_f16_fast_256x128_v1, DT_F16, 256, 128, 2, 2, A_CONV, B_KN, 8, 1)
TILE_KERNEL(mtk_conv_f16_fast_128x128_v8, DT_F16, 128, 128, 2, 2, A_CONV, B_KN, 8, 8)
TILE_KERNEL(mtk_conv_f16_fast_128x128_v4, DT_F16, 128, 128, 2, 2, A_CONV, B_KN, 8, 4)
TILE_KERNEL(mtk_conv_f16_fast_128x128_v1, DT_F16, 128, 128, 2, 2, A_CONV, B_KN, 8, 1)
TILE_KERNEL(mtk_conv_f16_gen_128x128_v8, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 8, 8)
TILE_KERNEL(mtk_conv_f16_gen_128x128_v4, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 4, 4)
TILE_KERNEL(mtk_conv_f16_gen_128x128_v1, DT_F16, 128, 128, 2, 2, A_CONV_GENERIC, B_KN, 1, 1)
