// fp16 tile-GEMM instantiations (reference default B layout [N][K] = "nt", and [K][N] = "nn"),
// plus the split-K second pass. Kernel names are what the runtime's kernel-select looks up.
#include "tile_gemm.hpp"

using namespace mtk;

#define TILE_KERNEL(NAME, DT, BM, BN, WM, WN, AK, BKIND, VA, VB)                    \
  extern "C" __global__ void __launch_bounds__(256) NAME(const mtk_tile_args a) { \
    tile_gemm<DT, BM, BN, WM, WN, AK, BKIND, VA, VB>(a);                          \
  }

#define GEMM_SET(DTN, DT)                                                                \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_256x256_v8, DT, 256, 256, 2, 2, A_MK, B_NK, 8, 8)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_256x256_v4, DT, 256, 256, 2, 2, A_MK, B_NK, 4, 4)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_256x256_v1, DT, 256, 256, 2, 2, A_MK, B_NK, 1, 1)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_128x128_v8, DT, 128, 128, 2, 2, A_MK, B_NK, 8, 8)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_128x128_v4, DT, 128, 128, 2, 2, A_MK, B_NK, 4, 4)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nt_128x128_v1, DT, 128, 128, 2, 2, A_MK, B_NK, 1, 1)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_256x256_v8, DT, 256, 256, 2, 2, A_MK, B_KN, 8, 8)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_256x256_v4, DT, 256, 256, 2, 2, A_MK, B_KN, 4, 4)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_256x256_v1, DT, 256, 256, 2, 2, A_MK, B_KN, 1, 1)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_128x128_v8, DT, 128, 128, 2, 2, A_MK, B_KN, 8, 8)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_128x128_v4, DT, 128, 128, 2, 2, A_MK, B_KN, 4, 4)     \
  TILE_KERNEL(mtk_gemm_##DTN##_nn_128x128_v1, DT, 128, 128, 2, 2, A_MK, B_KN, 1, 1)     \
  extern "C" __global__ void __launch_bounds__(256) mtk_splitk_reduce_##DTN(const mtk_reduce_args a) { \
    splitk_reduce<DT>(a);                                                                \
  }

GEMM_SET(f16, DT_F16)
