// GEMM kernel instantiations for one element type. A translation unit defines
//   MTK_GEMM_DT        DT_F16 or DT_BF16
//   MTK_GEMM_NAME(x)   the kernel name for suffix x (mtk_gemm_f16_##x, mtk_gemm_bf16_##x)
//   MTK_REDUCE_NAME    the split-K second pass (mtk_splitk_reduce_f16 / _bf16)
// and includes this file once. Kernel names are what the runtime's kernel-select looks up:
//   *_nt_*_d   B [N][K] (the reference's default layout), direct-to-LDS pipeline
//   *_nn_*_d   B [K][N] (config 1 "C = A.B row-major"), direct-to-LDS + transposed LDS reads
//   *_tt_*_d, *_tn_*_d   A [K][M] (the reference's transpose.left) with B [N][K] / [K][N]
//   *_s        split-K with the partitions run in sequence by one workgroup per tile
//   *_v1       2-byte register-staged fallback for odd leading dimensions
#pragma once

#include "tile_direct.hpp"

// 256x256 tiles: 8 wavefronts (2 x 4, 128 x 64 each, two per SIMD); 128x128: 4 (2 x 2).
#define MTK_DIRECT_KERNEL(SUFFIX, BM, BN, WM, WN, AOP, BOP, SER)                                              \
  extern "C" __global__ void __launch_bounds__(64 * WM * WN) MTK_GEMM_NAME(SUFFIX)(const mtk_tile_args a) { \
    mtk::tile_direct<MTK_GEMM_DT, BM, BN, WM, WN, AOP, BOP, SER>(a);                                        \
  }

#define MTK_TILE_KERNEL(SUFFIX, BM, BN, WM, WN, AK, BKIND, VA, VB)                             \
  extern "C" __global__ void __launch_bounds__(256) MTK_GEMM_NAME(SUFFIX)(const mtk_tile_args a) { \
    mtk::tile_gemm<MTK_GEMM_DT, BM, BN, WM, WN, mtk::AK, mtk::BKIND, VA, VB>(a);                \
  }

namespace mtk_gemm_ops {
using R256 = mtk::OpRows<256, 8>;
using C256 = mtk::OpColsT<256, 8>;
using R128 = mtk::OpRows<128, 4>;
using C128 = mtk::OpColsT<128, 4>;
}  // namespace mtk_gemm_ops

MTK_DIRECT_KERNEL(nt_256x256_d, 256, 256, 2, 4, mtk_gemm_ops::R256, mtk_gemm_ops::R256, false)
MTK_DIRECT_KERNEL(nt_128x128_d, 128, 128, 2, 2, mtk_gemm_ops::R128, mtk_gemm_ops::R128, false)
MTK_DIRECT_KERNEL(nt_256x256_s, 256, 256, 2, 4, mtk_gemm_ops::R256, mtk_gemm_ops::R256, true)
MTK_DIRECT_KERNEL(nt_128x128_s, 128, 128, 2, 2, mtk_gemm_ops::R128, mtk_gemm_ops::R128, true)
MTK_DIRECT_KERNEL(nn_256x256_d, 256, 256, 2, 4, mtk_gemm_ops::R256, mtk_gemm_ops::C256, false)
MTK_DIRECT_KERNEL(nn_128x128_d, 128, 128, 2, 2, mtk_gemm_ops::R128, mtk_gemm_ops::C128, false)
MTK_DIRECT_KERNEL(nn_256x256_s, 256, 256, 2, 4, mtk_gemm_ops::R256, mtk_gemm_ops::C256, true)
MTK_DIRECT_KERNEL(nn_128x128_s, 128, 128, 2, 2, mtk_gemm_ops::R128, mtk_gemm_ops::C128, true)
MTK_DIRECT_KERNEL(tt_256x256_d, 256, 256, 2, 4, mtk_gemm_ops::C256, mtk_gemm_ops::R256, false)
MTK_DIRECT_KERNEL(tt_128x128_d, 128, 128, 2, 2, mtk_gemm_ops::C128, mtk_gemm_ops::R128, false)
MTK_DIRECT_KERNEL(tt_256x256_s, 256, 256, 2, 4, mtk_gemm_ops::C256, mtk_gemm_ops::R256, true)
MTK_DIRECT_KERNEL(tt_128x128_s, 128, 128, 2, 2, mtk_gemm_ops::C128, mtk_gemm_ops::R128, true)
MTK_DIRECT_KERNEL(tn_256x256_d, 256, 256, 2, 4, mtk_gemm_ops::C256, mtk_gemm_ops::C256, false)
MTK_DIRECT_KERNEL(tn_128x128_d, 128, 128, 2, 2, mtk_gemm_ops::C128, mtk_gemm_ops::C128, false)
MTK_DIRECT_KERNEL(tn_256x256_s, 256, 256, 2, 4, mtk_gemm_ops::C256, mtk_gemm_ops::C256, true)
MTK_DIRECT_KERNEL(tn_128x128_s, 128, 128, 2, 2, mtk_gemm_ops::C128, mtk_gemm_ops::C128, true)

MTK_TILE_KERNEL(nt_256x256_v1, 256, 256, 2, 2, A_MK, B_NK, 1, 1)
MTK_TILE_KERNEL(nt_128x128_v1, 128, 128, 2, 2, A_MK, B_NK, 1, 1)
MTK_TILE_KERNEL(nn_256x256_v1, 256, 256, 2, 2, A_MK, B_KN, 1, 1)
MTK_TILE_KERNEL(nn_128x128_v1, 128, 128, 2, 2, A_MK, B_KN, 1, 1)

extern "C" __global__ void __launch_bounds__(256) MTK_REDUCE_NAME(const mtk_reduce_args a) {
  mtk::splitk_reduce<MTK_GEMM_DT>(a);
}
